"""The allocation-free entry point (dkv_attend_layer_noalloc: the K1 decode and one layer with
the library's static workspace) against the existing entry points with a caller workspace
(dkv_attend_prepare + dkv_attend_layer): identical outputs on calls in a row, the second
context smaller than the first, so it runs over what the first left in the static array; and
the same calls captured in a HIP graph (after the first, eager call on the device)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _workload(tokens: int, seed: int):
    import synth
    import workloads

    shape = synth.ModelShape(2, 8, 64, 32, 1024)  # Llama-3.2-1B shape, two layers
    return workloads.build_decode("noalloc", shape=shape, tokens=tokens, seed=seed, device=DEV,
                                  query_dtype=torch.float32, query_scale=100.0)


def _with_workspace(w) -> torch.Tensor:
    import dkv_hip

    dkv_hip.attend_prepare(w.args[0], w.workspace)
    for a in w.args:
        dkv_hip.attend_layer(a, w.workspace)
    torch.cuda.synchronize()
    return w.outs.clone()


def test_noalloc_matches_workspace_entry_points():
    import dkv_hip

    print("[case] dkv_attend_layer_noalloc: 1B shape, 1,500 then 700 tokens", flush=True)
    big, small = _workload(1500, 11), _workload(700, 12)
    refs = [_with_workspace(w) for w in (big, small)]
    for w in (big, small):
        w.outs.fill_(float("nan"))
    torch.cuda.synchronize()
    for w in (big, small):  # calls in a row: the second, smaller context after the first
        for a in w.args:
            dkv_hip.attend_layer_noalloc(a)
    torch.cuda.synchronize()
    for w, ref, name in ((big, refs[0], "1,500 tokens"), (small, refs[1], "700 tokens")):
        assert torch.isfinite(w.outs).all(), name
        assert torch.equal(w.outs, ref), f"{name}: max abs diff {(w.outs - ref).abs().max().item():.3e}"
    # and once more on the bigger context after the smaller one
    big.outs.fill_(float("nan"))
    for a in big.args:
        dkv_hip.attend_layer_noalloc(a)
    torch.cuda.synchronize()
    assert torch.equal(big.outs, refs[0])


def test_noalloc_calls_replay_from_a_graph():
    """Two layers of dkv_attend_layer_noalloc recorded in one HIP graph, after an eager call on the
    device (the first call looks up the static array's address): every replay equals the
    workspace entry points' output bit for bit, with eager noalloc calls on another, larger
    context between the replays overwriting the static array."""
    import dkv_hip

    print("[case] dkv_attend_layer_noalloc under graph capture: 1B shape, 700 tokens", flush=True)
    w, other = _workload(700, 13), _workload(1500, 14)
    ref = _with_workspace(w)
    for a in w.args:  # eager: the device's array address is looked up here, outside any capture
        dkv_hip.attend_layer_noalloc(a)
    torch.cuda.synchronize()
    assert torch.equal(w.outs, ref)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for a in w.args:
            dkv_hip.attend_layer_noalloc(a)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for a in w.args:
            dkv_hip.attend_layer_noalloc(a)
    torch.cuda.synchronize()
    for rep in range(3):
        w.outs.fill_(float("nan"))
        for a in other.args:  # leaves the other context's workspace in the static array
            dkv_hip.attend_layer_noalloc(a)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(w.outs, ref), f"replay {rep}: max abs diff {(w.outs - ref).abs().max().item():.3e}"
