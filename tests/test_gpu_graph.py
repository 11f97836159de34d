"""A decode step recorded in a HIP graph and replayed gives the eager step's output exactly, on
every replay, with eager work and synchronisations between the replays."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_graph_replay_matches_eager():
    import workloads

    print("[case] graph replay of a 1b-1500 decode step", flush=True)
    w = workloads.build_decode("1b-1500", device="cuda")
    w.step()
    torch.cuda.synchronize()
    eager = w.outs.clone()
    graph = w.capture()
    for rep in range(4):
        w.outs.fill_(float("nan"))          # eager work between replays
        w.step() if rep == 2 else None      # and an eager step on the same buffers
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(w.outs, eager), f"replay {rep} differs from the eager step"
