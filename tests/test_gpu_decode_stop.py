"""GPU parity of the decode loop's stop-token check (language_model.cpp:643-671,
language_model_dflash.cpp:570-579, language_model_gemma4_mtp.cpp:940-956)
against the oracle: kept counts and stop reasons bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_stop_check_parity(gpu, oracle):
    import torch
    import llima_amd
    print("[gpu-case] stop check", flush=True)
    rng = np.random.default_rng(12)
    V = 128256
    stop = [128001, 128008, 128009, 7, 0]
    for B, M in [(1, 1), (64, 1), (16, 8), (300, 16), (5, 0)]:
        toks = rng.integers(-2, V + 3, size=(B, M)).astype(np.int32)
        hit = rng.random((B, M)) < 0.08
        toks[hit] = rng.choice(stop, hit.sum())
        count = rng.integers(0, M + 2, B).astype(np.int32)
        room = rng.integers(-1, M + 3, B).astype(np.int32)
        mask = llima_amd.stop_mask(stop, V, gpu)
        t = torch.from_numpy(toks).to(gpu)
        for c, r in ((None, None), (count, None), (count, room)):
            keep, status = llima_amd.stop_check(t, mask, V, None if c is None else torch.from_numpy(c),
                                                None if r is None else torch.from_numpy(r))
            ek, es = oracle.stop_check(toks, stop, count=c, room=r)
            assert (keep.cpu().numpy() == ek).all() and (status.cpu().numpy() == es).all(), (B, M)


def test_stop_check_room_filled_exactly(gpu):
    """A run that fills the cache room exactly reports the cache full, and a
    stop token at its last position still wins (language_model_gemma4_mtp.cpp:
    948-955, 1011-1012): hand-derived, as in the oracle's test."""
    import torch
    import llima_amd
    print("[gpu-case] stop check room == n", flush=True)
    V = 128256
    stop = [2, 128001, 128009]
    toks = torch.tensor([[5, 7, 2, 9], [128009, 1, 1, 1], [4, 4, 4, 4], [4, 4, 2, 4], [-1, 3, 2, 0]],
                        dtype=torch.int32, device=gpu)
    count = torch.tensor([2, 4, 4, 3, 0], dtype=torch.int32)
    room = torch.tensor([2, 1, 4, 3, 0], dtype=torch.int32)
    keep, status = llima_amd.stop_check(toks, llima_amd.stop_mask(stop, V, gpu), V, count, room)
    assert keep.cpu().tolist() == [2, 1, 4, 3, 0]
    assert status.cpu().tolist() == [2, 1, 2, 1, 2]
