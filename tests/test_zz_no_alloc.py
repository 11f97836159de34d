"""The allocation-free entry point (dkv_attend_layer_noalloc: the K1 decode and one layer with
the library's static workspace) against the existing entry points with a caller workspace
(dkv_attend_prepare + dkv_attend_layer): identical outputs on calls in a row, the second
context smaller than the first, so it runs over what the first left in the static array."""

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
