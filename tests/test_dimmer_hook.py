"""CPU checks of the ``dimmer`` attention hook's eager path (scripts/dimmer.py:45-129): a tiny random
Llama built from a local config (nothing downloaded) must give the same logits through the hook as
through transformers' own eager attention; captured scores must satisfy what softmax fixes (each
query hands out exactly one unit of attention, so the H2O sums over keys equal queries x groups
and the SnapKV sums equal window x groups); chunked prefill must capture the same scores as one
pass; an evicted slot must receive no attention."""

from __future__ import annotations

import pytest
import torch

import synth

SHAPE = synth.ModelShape(2, 2, 16, 4, 32)  # 2 layers, 2 KV heads x 16, 4 query heads (2 per KV head)


def _model(seed: int):
    from transformers import LlamaForCausalLM

    torch.manual_seed(seed)
    config = synth.llama_config(SHAPE)
    config.vocab_size, config.intermediate_size = 64, 32
    return LlamaForCausalLM(config).float().eval()


def _ids(tokens: int, seed: int) -> torch.Tensor:
    return torch.randint(0, 64, (1, tokens), generator=torch.Generator().manual_seed(seed))


def test_hook_logits_match_transformers_eager():
    import dimmer

    model = _model(0)
    ids = _ids(40, 1)
    model.set_attn_implementation("eager")
    with torch.no_grad():
        want = model(input_ids=ids).logits
    dimmer.install(model)
    with torch.no_grad():
        got = model(input_ids=ids).logits
    assert torch.allclose(got, want, atol=1e-5, rtol=1e-5), float((got - want).abs().max())


@pytest.mark.parametrize("chunk", [16, 512])
def test_prefill_scores_sum_to_query_counts(chunk):
    import dimmer

    model = _model(1)
    dimmer.install(model)
    tokens, window, groups = 70, 8, SHAPE.q_heads // SHAPE.kv_heads
    with torch.no_grad():
        cache, scores = dimmer.prefill_with_scores(model, _ids(tokens, 2), window=window, chunk=chunk)
    assert cache.get_seq_length() == tokens
    for total, snap in zip(scores["sum"], scores["snap"]):
        assert total.shape == snap.shape == (SHAPE.kv_heads, tokens)
        torch.testing.assert_close(total.sum(dim=1), torch.full((SHAPE.kv_heads,), float(tokens * groups)))
        torch.testing.assert_close(snap.sum(dim=1), torch.full((SHAPE.kv_heads,), float(window * groups)))
        # causal: the last token is seen by the last query only (per head, ``groups`` query heads)
        assert (total[:, -1] <= groups + 1e-4).all()


def test_chunked_prefill_scores_equal_one_pass():
    import dimmer

    model = _model(2)
    dimmer.install(model)
    ids = _ids(75, 3)  # 75 = 4 chunks of 16 + 11, the short tail (< window 12) merges into the 4th
    assert dimmer._chunk_bounds(75, 16, 12) == [0, 16, 32, 48, 75]
    with torch.no_grad():
        _, one = dimmer.prefill_with_scores(model, ids, window=12, chunk=512)
        _, many = dimmer.prefill_with_scores(model, ids, window=12, chunk=16)
    for kind in ("sum", "snap"):
        for a, b in zip(one[kind], many[kind]):
            torch.testing.assert_close(a, b, atol=1e-4, rtol=1e-4)
    means = dimmer.mean_scores(one["sum"])
    tokens = ids.shape[1]
    torch.testing.assert_close(means[0][:, 0], one["sum"][0][:, 0] / tokens)
    torch.testing.assert_close(means[0][:, -1], one["sum"][0][:, -1])


def test_evicted_slots_receive_no_attention():
    import dimmer

    model = _model(3)
    dimmer.install(model)
    ids = _ids(30, 4)
    with torch.no_grad():
        cache = model(input_ids=ids, use_cache=True).past_key_values
    evicted = [torch.zeros(SHAPE.kv_heads, 30, dtype=torch.bool) for _ in range(SHAPE.layers)]
    evicted[0][1, 5:12] = True
    dimmer.set_eviction(evicted)
    dimmer.STATE.scores, dimmer.STATE.window_scores, dimmer.STATE.window = {}, {}, 2
    dimmer.STATE.scoring = True
    try:
        with torch.no_grad():
            model(input_ids=_ids(2, 5), past_key_values=cache, position_ids=torch.tensor([[30, 31]]),
                  use_cache=True)
    finally:
        dimmer.STATE.scoring = False
        dimmer.set_eviction(None)
    received = dimmer.STATE.scores[0]
    assert received.shape == (SHAPE.kv_heads, 32)
    assert float(received[1, 5:12].abs().max()) == 0.0
    assert float(received[0, 5:12].min()) > 0.0
    assert float(dimmer.STATE.scores[1][:, 5:12].min()) > 0.0
