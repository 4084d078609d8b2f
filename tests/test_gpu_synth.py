"""The device generator writes exactly the bytes of its host twin
(breadv2_amd/synth.py), so host-side fixtures and device-resident weights
agree without copying."""
import numpy as np
import pytest
import torch

from breadv2_amd import api, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("n_blocks,seed", [(1, 0), (3, 1), (1000, 42), (4097, 2**40 + 7)])
def test_synth_q4k_matches_host(n_blocks, seed):
    t = torch.empty(n_blocks * 144, dtype=torch.uint8, device=DEV)
    api.synth_q4k(t, n_blocks, seed)
    assert np.array_equal(t.cpu().numpy(), synth.synth_q4k(n_blocks, seed))


@pytest.mark.parametrize("n_blocks,seed", [(1, 0), (3, 1), (1001, 42), (4097, 2**40 + 7)])
def test_synth_q6k_matches_host(n_blocks, seed):
    # odd block counts leave a 2-byte tail that is not a whole dword
    t = torch.full((n_blocks * 210 + 2,), 0xAB, dtype=torch.uint8, device=DEV)
    api.synth_q6k(t, n_blocks, seed)
    got = t.cpu().numpy()
    assert np.array_equal(got[: n_blocks * 210], synth.synth_q6k(n_blocks, seed))
    assert np.all(got[n_blocks * 210:] == 0xAB)


def test_synth_normal_moments():
    n = 1 << 20
    t = torch.empty(n, dtype=torch.float32, device=DEV)
    api.synth_normal_f32(t, n, 5, 0.0, 0.02)
    x = t.cpu().numpy().astype(np.float64)
    assert abs(x.mean()) < 1e-4
    assert abs(x.std() - 0.02) < 2e-4
