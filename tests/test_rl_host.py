"""RL plumbing on the CPU: the rollout buffer contract (reference
``tests/rl/test_zero_copy_rollout.py`` CPU cases and ``rl/rollout.py``
errors) and the packed-pixel helpers against brute force."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gbxcule_amd.rl import (
    RolloutBuffer,
    get_diff_lut,
    get_unpack_lut,
    pack_2bpp_u8,
    packed_l1_distance,
    unpack_2bpp_u8,
)


def _rb(**kw):
    args = dict(steps=8, num_envs=4, stack_k=1, obs_format="packed2", device="cpu")
    args.update(kw)
    return RolloutBuffer(**args)


def _fields(n, fill=0):
    return dict(
        actions=torch.full((n,), fill, dtype=torch.int32),
        rewards=torch.full((n,), float(fill), dtype=torch.float32),
        dones=torch.zeros(n, dtype=torch.bool),
        values=torch.zeros(n, dtype=torch.float32),
        logprobs=torch.zeros(n, dtype=torch.float32),
    )


def test_obs_slot_is_a_view():
    r = _rb(steps=16)
    slot = r.obs_slot(10)
    assert slot.shape == (4, 1, 72, 20) and slot.is_contiguous()
    slot.fill_(42)
    assert r.obs[10].sum().item() == 42 * slot.numel()
    for i in range(16):
        assert r.obs_slot(i).is_contiguous()
    with pytest.raises(ValueError):
        r.obs_slot(16)


def test_set_step_fields_and_batch():
    r = _rb(steps=3, obs_steps=4)
    for t in range(3):
        f = _fields(4, fill=t + 1)
        r.set_step_fields(t, **f)
    assert r.step == 3
    assert r.actions[2].tolist() == [3] * 4 and r.rewards[1].sum().item() == 8.0
    b = r.as_batch()
    assert b["obs_u8"].shape == (12, 1, 72, 20) and b["actions"].shape == (12,)
    assert r.as_batch(flatten_obs=False)["obs_u8"].shape == (3, 4, 1, 72, 20)
    bad = _fields(4)
    bad["actions"] = bad["actions"].to(torch.int64)
    with pytest.raises(ValueError, match="actions: expected dtype"):
        r.set_step_fields(0, **bad)
    with pytest.raises(ValueError, match="step_idx"):
        r.set_step_fields(3, **_fields(4))


def test_add_and_errors():
    r = _rb(steps=2, obs_format="u8", height=4, width=8)
    obs = torch.ones((4, 1, 4, 8), dtype=torch.uint8)
    r.add(obs, **_fields(4))
    r.add(obs * 2, **_fields(4))
    assert r.obs[1].max().item() == 2
    with pytest.raises(RuntimeError, match="full"):
        r.add(obs, **_fields(4))
    with pytest.raises(RuntimeError, match="not full"):
        _rb().as_batch()
    for kw, msg in ((dict(steps=0), "steps"), (dict(num_envs=0), "num_envs"),
                    (dict(stack_k=0), "stack_k"), (dict(obs_format="rgb"), "obs_format"),
                    (dict(width=21), "packed2 frames"), (dict(obs_steps=2), "obs_steps")):  # fmt: skip
        with pytest.raises(ValueError, match=msg):
            _rb(**kw)


def test_pack_unpack_roundtrip():
    g = torch.Generator().manual_seed(3)
    px = torch.randint(0, 4, (5, 72, 80), generator=g, dtype=torch.uint8)
    packed = pack_2bpp_u8(px)
    assert packed.shape == (5, 72, 20)
    # leftmost pixel in bits 0-1
    assert int(packed[0, 0, 0]) == int(px[0, 0, 0]) | int(px[0, 0, 1]) << 2 | int(
        px[0, 0, 2]
    ) << 4 | int(px[0, 0, 3]) << 6
    assert torch.equal(unpack_2bpp_u8(packed), px)
    assert torch.equal(unpack_2bpp_u8(packed, lut=get_unpack_lut()), px)


def test_diff_lut_brute_force():
    lut = get_diff_lut().numpy()
    for a in range(0, 256, 7):
        for b in range(0, 256, 5):
            want = sum(abs(((a >> (2 * k)) & 3) - ((b >> (2 * k)) & 3)) for k in range(4))
            assert lut[a, b] == want


def test_packed_l1_distance():
    g = torch.Generator().manual_seed(4)
    obs = torch.randint(0, 256, (6, 1, 72, 20), generator=g, dtype=torch.uint8)
    goal = torch.randint(0, 256, (1, 72, 20), generator=g, dtype=torch.uint8)
    d = packed_l1_distance(obs, goal)
    lut = get_diff_lut()
    want = lut[obs.long(), goal.unsqueeze(0).long()].float().sum(dim=(1, 2, 3)) / (72 * 80 * 3)
    assert torch.equal(d, want)
    zeros = torch.zeros((2, 1, 72, 20), dtype=torch.uint8)
    assert packed_l1_distance(zeros, zeros[0]).tolist() == [0.0, 0.0]
    assert packed_l1_distance(zeros, torch.full((1, 72, 20), 0xFF, dtype=torch.uint8)).tolist() == [1.0, 1.0]
    with pytest.raises(ValueError):
        packed_l1_distance(zeros.float(), zeros[0])
    with pytest.raises(ValueError):
        packed_l1_distance(zeros, torch.zeros((1, 72, 19), dtype=torch.uint8))
    # one goal per env ([N, 1, H, W_bytes]): each env against its own goal
    goals = torch.randint(0, 256, (6, 1, 72, 20), generator=g, dtype=torch.uint8)
    per = packed_l1_distance(obs, goals)
    want = lut[obs.long(), goals.long()].float().sum(dim=(1, 2, 3)) / (72 * 80 * 3)
    assert torch.equal(per, want)
    assert torch.equal(packed_l1_distance(obs, goal.unsqueeze(0)), d)  # [1, 1, H, W_bytes]
    for bad in ((72, 20), (2, 2, 72, 20), (4, 1, 72, 20), (1, 1, 1, 72, 20)):
        with pytest.raises(ValueError):
            packed_l1_distance(obs, torch.zeros(bad, dtype=torch.uint8))
    # uniform shades: E|a - b| = 20 / 16 over the 16 pairs, normalised by 3
    assert np.isclose(float(d.mean()), 20 / 16 / 3, atol=0.02)
