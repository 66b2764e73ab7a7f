"""EnvMemoryView indexing semantics on the CPU.

The view stands for the reference's env-major ``memory_torch()``
(``backends/warp_vec.py:799-810``).  Here its rectangle reads and writes go to
a plain ``[N, 65536]`` CPU tensor, and every index must give exactly what the
same index gives on that tensor: shapes, dtypes, values, and for assignment
the memory afterwards.  The expressions of the reference's RL callers
(``rl/pokered_packed_parcel_env.py:277-291, 388-391``) are among the keys.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gbxcule_amd.memview import EnvMemoryView

N = 70  # not a multiple of 64


def _make(seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    store = torch.randint(0, 256, (N, 65536), dtype=torch.uint8, generator=g)
    calls = {"read": 0, "write": 0}

    def read(e0, e1, a0, a1):
        calls["read"] += 1
        return store[e0:e1, a0:a1].clone()

    def write(e0, e1, a0, a1, src):
        calls["write"] += 1
        assert src.shape == (e1 - e0, a1 - a0) and src.dtype == torch.uint8
        store[e0:e1, a0:a1] = src

    return EnvMemoryView(N, torch.device("cpu"), read, write), store, calls


KEYS = [
    (slice(None), 0xD35E),
    (slice(None), slice(0xD747, 0xD747 + 320)),
    (0, 0xD35E),
    (5, slice(0xC000, 0xC010)),
    (-1, slice(0xFF00, 0x10000)),
    3,
    (slice(2, 9), slice(0x8000, 0x8040, 4)),
    (slice(None, None, 3), -1),
    (torch.tensor([4, 1, 66]), 0xFF40),
    (torch.tensor([4, 1, 66]), torch.tensor([0xFF40, 0xC000, 7])),
    ([0, 2], slice(100, 110)),
    (torch.arange(N) % 3 == 0, 0xC123),
    (Ellipsis, 0xFF44),
    (slice(None), slice(10, 10)),
    (slice(None), torch.tensor(0xFF41)),
]


def test_is_a_uint8_tensor_of_the_reference_shape():
    v, store, _ = _make()
    assert isinstance(v, torch.Tensor)
    assert v.dtype is torch.uint8 and v.ndim == 2 and tuple(v.shape) == (N, 65536)
    assert v.size(0) == N and v.dim() == 2 and len(v) == N and v.numel() == N * 65536


@pytest.mark.parametrize("k", range(len(KEYS)))
def test_getitem_matches_env_major(k):
    v, store, calls = _make(k)
    key = KEYS[k]
    got, want = v[key], store[key]
    assert type(got) is torch.Tensor
    assert got.shape == want.shape and got.dtype == want.dtype
    assert torch.equal(got, want)
    assert calls["read"] == 1  # one rectangle read per index


@pytest.mark.parametrize("k", range(len(KEYS)))
def test_setitem_matches_env_major(k):
    v, store, _ = _make(100 + k)
    ref = store.clone()
    key = KEYS[k]
    shape = ref[key].shape
    g = torch.Generator().manual_seed(k)
    val = torch.randint(0, 256, shape, dtype=torch.uint8, generator=g)
    v[key] = val
    ref[key] = val
    assert torch.equal(store, ref)
    v[key] = 7  # scalar broadcast
    ref[key] = 7
    assert torch.equal(store, ref)


def test_inplace_or_through_index_is_the_lcdc_override():
    # reference warp_vec.py:734-757: set LCDC bit 7, keep the other bits
    v, store, calls = _make(3)
    ref = store.clone()
    v[:, 0xFF40] |= 0x80
    ref[:, 0xFF40] |= 0x80
    assert torch.equal(store, ref)
    assert calls == {"read": 1, "write": 1}


def test_other_ops_run_on_a_copy_and_inplace_ops_write_back():
    v, store, _ = _make(4)
    assert torch.equal(v.clone(), store)
    assert int(v.sum()) == int(store.sum())
    assert torch.equal((v[:, 0x100] > 128), store[:, 0x100] > 128)
    v.zero_()
    assert int(store.abs().sum()) == 0


def test_index_errors_like_torch():
    v, store, _ = _make(5)
    for key in [(N, 0), (0, 65536), (-N - 1, 0), (0, 0, 0)]:
        with pytest.raises(IndexError):
            v[key]
        with pytest.raises(IndexError):
            store[key]
    with pytest.raises(IndexError):
        v[torch.tensor([0, N]), 5]
    with pytest.raises(IndexError):
        v[0, torch.tensor([1.0])]


def test_reference_rl_expressions():
    # rl/pokered_packed_parcel_env.py:388-391 and :277-291
    v, store, _ = _make(6)
    events = v[:, 0xD747 : 0xD747 + 320]
    assert events.shape == (N, 320) and torch.equal(events, store[:, 0xD747:0xD887])
    for addr in (0xD35E, 0xD362, 0xD361):
        x = v[:, addr]
        assert x.shape == (N,) and torch.equal(x, store[:, addr])
        assert torch.equal(x.float(), store[:, addr].float())
    assert int(v[0, 0xD35E].item()) == int(store[0, 0xD35E])
    np.testing.assert_array_equal(v[0, 0xD747:0xD757].numpy(), store[0, 0xD747:0xD757].numpy())


def test_full_copy_warns_once_above_threshold(monkeypatch):
    """Operations that copy all memory warn once per view when the copy is
    large; indexing never does."""
    import warnings

    import gbxcule_amd.memview as mv

    mem, store, _ = _make(3)
    monkeypatch.setattr(mv, "FULL_COPY_WARN_BYTES", N * 65536 - 1)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        mem[:, 0xD35E]
        mem[5, 0xC000:0xC010]
    with pytest.warns(mv.FullCopyWarning):
        total = mem.sum()
    assert int(total) == int(store.sum())
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        (mem == 7).any(1)  # second full copy: no second warning
    monkeypatch.setattr(mv, "FULL_COPY_WARN_BYTES", N * 65536)
    fresh, _, _ = _make(4)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        fresh.sum()  # at the threshold: no warning
