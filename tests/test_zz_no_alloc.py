"""ppo_epoch_permutations_noalloc (the permutation entry point whose
workspace is the library's own device scratch) against
ppo_epoch_permutations with a caller-owned workspace, through the C ABI: two
calls in a row, the second with a smaller input (the scratch keeps the first
call's contents), both bit-exact; a size beyond the scratch is rejected on the
host before anything is launched."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib

pytestmark = pytest.mark.gpu

PPO_ERR_SPACE = -3


def _with_workspace(key, epochs, n):
    lib = _lib.load()
    ws = torch.zeros(lib.ppo_epoch_permutations_workspace(epochs, n), dtype=torch.uint8, device="cuda")
    out = torch.full((epochs, n), -1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("ppo_epoch_permutations", st, key.data_ptr(), epochs, n, out.data_ptr(), ws.data_ptr(), ws.numel())
    return out


def _noalloc(key, epochs, n):
    out = torch.full((epochs, n), -1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("ppo_epoch_permutations_noalloc", st, key.data_ptr(), epochs, n, out.data_ptr())
    return out


def test_noalloc_permutations_equal_the_workspace_entry_point():
    # the discrete Anakin update's 4 epochs of 262144 samples, then the
    # recurrent update's 4 epochs of 1024 envs (a smaller input over a
    # scratch that still holds the first call's buckets)
    for seed, epochs, n in ((3, 4, 262144), (9, 4, 1024)):
        print(f"noalloc permutations: seed {seed}, {epochs} epochs of {n}", flush=True)
        key = torch.tensor([0, seed], dtype=torch.int32, device="cuda")
        got = _noalloc(key, epochs, n)
        want = _with_workspace(key, epochs, n)
        torch.cuda.synchronize()
        g = got.cpu().numpy()
        assert np.array_equal(g, want.cpu().numpy())
        assert all(np.array_equal(np.sort(row), np.arange(n)) for row in g)


def test_noalloc_rejects_a_size_beyond_its_scratch():
    lib = _lib.load()
    key = torch.zeros(2, dtype=torch.int32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    n = 1 << 22   # 4 epochs of 4M items need about 260 MB of workspace
    assert lib.ppo_epoch_permutations_workspace(4, n) > 24 << 20
    rc = lib.ppo_epoch_permutations_noalloc(st, key.data_ptr(), 4, n, out.data_ptr())
    assert rc == PPO_ERR_SPACE
    assert b"scratch" in lib.ppo_last_error()
    lib.ppo_clear_error()
