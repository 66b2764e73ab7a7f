"""The RL rollout pattern on the device, replayed on the oracle: savestate
start, snapshot broadcast, step -> packed render into rollout slots -> RAM
senses -> reward/termination -> masked reset, on a non-default stream.  Also
the reference's render-contract tests (``tests/rl/test_render_contract.py``)
and a double-buffer hand-off between an actor and a learner stream."""

from __future__ import annotations

import contextlib

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from ._parity import assert_same_state, ref_export_env, ref_import_env
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

SENSES = [0xC000, 0xC001, 0xC010, 0xFF40, 0xFF44, 0xFF80]


def _oracle_reward(frame: np.ndarray, start: np.ndarray) -> np.ndarray:
    """packed_l1_distance restated on unpacked shades."""
    def unpack(p):
        return np.stack([(p >> (2 * k)) & 3 for k in range(4)], -1).astype(np.int32)

    d = np.abs(unpack(frame) - unpack(start)[None]).reshape(frame.shape[0], -1).sum(1)
    return (d.astype(np.float32) / np.float32(72 * 80 * 3)).astype(np.float32)


def test_rollout_matches_oracle_replay(carts, bootstub, tmp_path):
    require_gpu()
    import torch

    from gbxcule_amd.abi import parse_cartridge_header
    from gbxcule_amd.backend import HipVecBackend
    from gbxcule_amd.rl import PackedPixelEnv, RolloutBuffer, collect_rollout, packed_l1_distance
    from gbxcule_amd.state_io import apply_state_to_image, load_pyboy_state

    rom = carts["c5"]
    n, fs, steps, max_steps = 64, 24, 7, 3
    # a savestate from a short run of another backend
    pre = HipVecBackend(rom, num_envs=4, frames_per_step=fs, stage="emulate_only", bootrom=bootstub)
    pre.reset(seed=0)
    for k in range(2):
        pre.step(seeded_actions(9, k, 4))
    path = tmp_path / "start.state"
    pre.save_state_file(str(path), env_idx=1)
    pre.close()

    def reward_fn(env, pixels, senses):
        reward = packed_l1_distance(pixels, env.start_pixels)
        return reward, (senses[:, 0] & 1) == 1

    env = PackedPixelEnv(rom, state_path=str(path), num_envs=n, frames_per_step=fs,
                         max_steps=max_steps, sense_addrs=SENSES, reward_fn=reward_fn,
                         bootrom=bootstub)  # fmt: skip
    ref = RefMachine(n, rom, bootstub)
    try:
        obs = env.reset(seed=0)
        # oracle: load into env 0, render (LCD forced on), snapshot, broadcast
        img = ref_export_env(ref, 0)
        ram = parse_cartridge_header(rom).ram_byte_length
        apply_state_to_image(load_pyboy_state(path, expected_cart_ram_size=ram), img)
        ref_import_env(ref, 0, img)
        ref.mem[:, 0xFF40] |= 0x80
        ref.render(packed=True)
        start = ref.pix_packed[0].copy()
        ref.snapshot(0)
        ref.masked_reset(np.ones(n, np.uint8))
        np.testing.assert_array_equal(env.start_pixels.cpu().numpy()[0], start)
        np.testing.assert_array_equal(obs["pixels"].cpu().numpy()[:, 0], np.broadcast_to(start, (n, 72, 20)))
        np.testing.assert_array_equal(obs["senses"].cpu().numpy(), ref.mem[:, SENSES])
        assert_same_state(env.backend, ref, step=-1, tag="rl reset")

        acts = [torch.from_numpy(seeded_actions(5, t, n)).cuda() for t in range(steps)]
        zeros = torch.zeros(n, dtype=torch.float32, device="cuda")
        calls = []

        def policy(o):
            calls.append(o.data_ptr())
            return acts[len(calls) - 1], zeros, zeros

        rollout = RolloutBuffer(steps=steps, num_envs=n, stack_k=1, obs_format="packed2",
                                obs_steps=steps + 1, device="cuda")  # fmt: skip
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            collect_rollout(env, policy, rollout)
        stream.synchronize()
        # every policy call saw the previous step's rollout slot (no copies)
        assert calls == [rollout.obs_slot(t).data_ptr() for t in range(steps)]

        ep = np.zeros(n, np.int32)
        resets = 0
        for t in range(steps):
            a = seeded_actions(5, t, n)
            ref.step(a, fs, 8, "emulate_only", threads=8)
            ref.mem[:, 0xFF40] |= 0x80
            ref.render(packed=True)
            frame = ref.pix_packed.copy()
            senses = ref.mem[:, SENSES].copy()
            ep += 1
            done = ((senses[:, 0] & 1) == 1) | (ep >= max_steps)
            reward = _oracle_reward(frame, start)
            ref.masked_reset(done.astype(np.uint8))
            ep[done] = 0
            frame[done] = start
            resets += int(done.sum())
            np.testing.assert_array_equal(rollout.obs[t + 1, :, 0].cpu().numpy(), frame, err_msg=f"t {t}")
            np.testing.assert_array_equal(rollout.dones[t].cpu().numpy(), done, err_msg=f"t {t}")
            np.testing.assert_array_equal(rollout.actions[t].cpu().numpy(), a)
            np.testing.assert_array_equal(rollout.rewards[t].cpu().numpy().view(np.uint32),
                                          reward.view(np.uint32), err_msg=f"t {t}")  # fmt: skip
        assert resets > n  # truncation alone resets every env twice in 7 steps
        np.testing.assert_array_equal(env.obs["senses"].cpu().numpy(), ref.mem[:, SENSES])
        assert_same_state(env.backend, ref, step=steps, tag="rl rollout")
    finally:
        env.close()
        ref.close()


def _contract_backend(rom, boot, **kw):
    from gbxcule_amd.backend import HipVecBackend

    args = dict(num_envs=1, frames_per_step=1, release_after_frames=1, render_pixels=False,
                render_pixels_packed=False, render_on_step=False, bootrom=boot)  # fmt: skip
    args.update(kw)
    return HipVecBackend(rom, **args)


def test_render_contract(carts, bootstub):
    """No implicit render with render_on_step=False; explicit render into a
    caller buffer and at a byte offset (reference test_render_contract.py)."""
    require_gpu()
    import torch

    rom = carts["c3"]
    b = _contract_backend(rom, bootstub, render_pixels=True)
    try:
        b.reset(seed=0)
        for _ in range(30):  # past the boot stub and into the drawn scene
            b.step_torch(torch.zeros((1,), dtype=torch.int32, device="cuda"))
        b.render_pixels_snapshot_torch()
        before = b.pixels_torch().clone()
        b.step_torch(torch.zeros((1,), dtype=torch.int32, device="cuda"))
        assert torch.equal(before, b.pixels_torch())
        out = torch.zeros((1, 1, 72, 20), dtype=torch.uint8, device="cuda")
        b.render_pixels_snapshot_packed_to_torch(out, 0)
        assert out.sum().item() > 0
        buf = torch.zeros((2, 1, 1, 72, 20), dtype=torch.uint8, device="cuda")
        b.render_pixels_snapshot_packed_to_torch(buf, 72 * 20)
        assert buf[0].sum().item() == 0 and torch.equal(buf[1], out)
        with pytest.raises(ValueError):
            b.render_pixels_snapshot_packed_to_torch(buf, 72 * 20 + 1)
    finally:
        b.close()


@contextlib.contextmanager
def _nothing():
    yield


def test_double_buffer_handoff(carts, bootstub):
    """Actor stream renders into buffer i and marks it ready; the learner
    stream waits on that event, consumes it and marks it free."""
    require_gpu()
    import torch

    from gbxcule_amd.rl import AsyncPPOBufferManager, RolloutBuffer

    rom = carts["c3"]
    n = 16
    b = _contract_backend(rom, bootstub, num_envs=n, frames_per_step=4)
    try:
        b.reset(seed=0)
        mgr = AsyncPPOBufferManager(num_buffers=2)
        bufs = [RolloutBuffer(steps=2, num_envs=n, stack_k=1, obs_format="packed2", obs_steps=3)
                for _ in range(2)]  # fmt: skip
        actor, learner = torch.cuda.Stream(), torch.cuda.Stream()
        seen = []
        act = torch.zeros((n,), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        for it in range(4):
            i = it % 2
            # iterations 0-1 call the hand-offs one by one, 2-3 as with-blocks
            with torch.cuda.stream(actor):
                if it < 2:
                    mgr.wait_free(i, actor)
                with mgr.filling(i, actor, policy_version=it) if it >= 2 else _nothing():
                    for t in range(3):
                        if t:
                            b.step_torch(act)
                        b.render_pixels_snapshot_packed_to_torch(bufs[i].obs_slot(t), 0)
                if it < 2:
                    mgr.mark_ready(i, actor, policy_version=it)
            with torch.cuda.stream(learner):
                if it < 2:
                    mgr.wait_ready(i, learner)
                    seen.append(bufs[i].obs.clone())
                    mgr.mark_free(i, learner)
                else:
                    with mgr.reading(i, learner):
                        seen.append(bufs[i].obs.clone())
        torch.cuda.synchronize()
        assert mgr.policy_version(1) == 3 and mgr.num_buffers == 2
        # consecutive hand-offs continue the same trajectory: the last frame
        # of one buffer is two steps before the first of the next
        for s in seen:
            assert s.shape == (3, n, 1, 72, 20)
        assert len({s.cpu().numpy().tobytes() for s in seen}) == 4
    finally:
        b.close()
