"""The committed fixtures of tests/golden/ (written by tests/golden/make_golden.py): the oracle must still produce
them (CPU), and the HIP library must reproduce them bit for bit (GPU)."""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _tiles(bits):
    z = np.load(os.path.join(GOLD, f"tiles_k{bits}.npz"))
    return z["words"], int(z["kin"]), int(z["n"]), z["weights"]


def _grouping_cases():
    z = np.load(os.path.join(GOLD, "grouping.npz"))
    for i in range(int(z["n"])):
        yield z[f"picks{i}"], int(z[f"count{i}"]), z[f"ids{i}"], z[f"members{i}"]


def test_codebook_fixture(oracle):
    want = np.load(os.path.join(GOLD, "codebook.npy"))
    assert want.shape == (65536,) and want.dtype == np.uint16
    assert np.array_equal(oracle.codebook_table(), want)
    # independent of the oracle: three states computed by hand from experts.rs:43-46
    for s in (0, 1, 0xFFFF):
        x = (s * 0xCBAC1FED) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = np.array([x & 0xFFFF], np.uint16).view(np.float16)[0]
        hi = np.array([x >> 16], np.uint16).view(np.float16)[0]
        v = np.float16(np.float32(lo) + np.float32(hi))
        assert want[s] == np.array([v], np.float16).view(np.uint16)[0], s


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_tile_fixture(oracle, bits):
    words, kin, n, want = _tiles(bits)
    assert np.array_equal(oracle.unpack(words, kin, n, bits), want)


def test_grouping_fixture(oracle):
    for picks, c, ids, mem in _grouping_cases():
        c2, ids2, mem2 = oracle.group(picks, picks.shape[0], 9, 289, 64)
        assert c2 == c and np.array_equal(ids2, ids) and np.array_equal(mem2, mem)


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_gpu_tiles_match_fixture(gfr, bits):
    import torch
    words, kin, n, want = _tiles(bits)
    w = torch.from_numpy(words.view(np.int32).reshape(kin // 16, n // 16, 8 * bits)).cuda()
    got = gfr.decode_tiles(w, kin, n, bits).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.gpu
def test_gpu_grouping_matches_fixture(gfr):
    import torch
    g = gfr.Grouping(289, 9, 64)
    for picks, c, ids, mem in _grouping_cases():
        g.members.fill_(12345)
        g.run(torch.from_numpy(picks).cuda(), picks.shape[0])
        torch.cuda.synchronize()
        assert int(g.count.item()) == c
        assert np.array_equal(g.ids[:c].cpu().numpy(), ids)
        assert np.array_equal(g.members.cpu().numpy(), mem)
