"""CPU checks of the synthetic workload draws: the fragmentation sweep's
geometric-run block ids (distinct, in range, disjoint restore targets, run
lengths with the requested mean, one sorted run for mean 640) and the
request batch's sizes."""

import numpy as np
import pytest

from pegaflow_amd import workload as wl


def _runs(ids):
    """Lengths of the maximal runs of consecutive increasing ids."""
    ids = np.asarray(ids)
    cuts = np.flatnonzero(np.diff(ids) != 1) + 1
    return np.diff(np.concatenate([[0], cuts, [len(ids)]]))


@pytest.mark.parametrize("mean", [1, 4, 32])
def test_draw_runs_distinct_and_mean(mean):
    rng = np.random.Generator(np.random.PCG64(7))
    lens = []
    for _ in range(40):
        ids = wl.draw_runs(rng, 20000, 600, mean)
        assert len(ids) == 600 and len(np.unique(ids)) == 600
        assert ids.min() >= 0 and ids.max() < 20000
        assert wl.run_count(ids) == len(_runs(ids))
        lens.append(_runs(ids))
    lens = np.concatenate(lens)
    # Geometric(1/mean) has mean `mean`; runs are cut at the request's end and
    # (rarely) at used blocks, and two runs can touch by chance.
    assert abs(lens.mean() - mean) / mean < 0.15, lens.mean()
    if mean == 1:
        # Geometric(1) is always 1: a run longer than 1 only forms by chance
        # adjacency, which at 600 of 20000 blocks is rare.
        assert (lens == 1).mean() > 0.9


def test_draw_runs_sorted_when_mean_covers_request():
    rng = np.random.Generator(np.random.PCG64(1))
    ids = wl.draw_runs(rng, 20000, 640, 640)
    assert np.array_equal(ids, np.arange(ids[0], ids[0] + 640))
    # With most of the tensor excluded, the window lands in the free part.
    mask = np.ones(1000, bool)
    mask[300:350] = False
    mask[700:720] = False
    ids = wl.draw_runs(rng, 1000, 50, 640, exclude=mask)
    assert np.array_equal(ids, np.arange(300, 350))
    with pytest.raises(ValueError, match="no free window"):
        wl.draw_runs(rng, 1000, 51, 640, exclude=mask)  # 70 free, no 51 in a row


def test_draw_runs_exclude_and_capacity():
    rng = np.random.Generator(np.random.PCG64(2))
    mask = np.zeros(200, bool)
    mask[::2] = True  # every even block taken
    ids = wl.draw_runs(rng, 200, 100, 4, exclude=mask)
    assert set(ids.tolist()) == set(range(1, 200, 2))  # exactly the free ones
    assert wl.run_count(ids) == 100  # no two odd blocks are adjacent
    with pytest.raises(ValueError, match="cannot draw"):
        wl.draw_runs(rng, 200, 101, 4, exclude=mask)


def test_fragmentation_requests_shape():
    reqs = wl.fragmentation_requests(20000, 4, seed=0, n_requests=16)
    again = wl.fragmentation_requests(20000, 4, seed=0, n_requests=16)
    sorted_reqs = wl.fragmentation_requests(20000, 640, seed=0, n_requests=16)
    assert len(reqs) == 16
    for (ids, targets), (ids2, t2), (sids, _) in zip(reqs, again, sorted_reqs):
        assert np.array_equal(ids, ids2) and np.array_equal(targets, t2)  # seeded
        assert 64 <= len(ids) <= 1024 and len(targets) == len(ids)
        assert len(sids) == len(ids)  # same token counts for every mean
        assert not set(ids.tolist()) & set(targets.tolist())
        assert len(np.unique(targets)) == len(targets)
        assert wl.run_count(sids) == 1
