"""End-to-end drop-in check through a Hugging Face Llama model (random weights, built from a local
config; nothing is downloaded), following the reference's direct-vs-rebuilt comparison
(scripts/test_compressed_attention.py:60-110): the same question is answered once over a rebuilt
cache with ordinary attention and once directly over the codes through the ``dimmer`` attention
hook (scripts/dimmer.py:45-48, 80-84) and ``greedy_answer`` (scripts/compressed_attention.py:140-169).
Both methods are covered: ``prog@b:r<f>`` (including question-time refinement scored over the codes,
scripts/methods.py:244-248) and ``dkvtc@b:snap:floor1``.

The two paths see the same codes, so their first-step logits must agree to the precision of the
direct path's fp16 key operands; the greedy replies must be the same."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPE = synth.ModelShape(2, 8, 64, 32, 1024)  # 2 layers, 8 KV heads x 64, 32 query heads, full-rank basis


class _Tokenizer:
    eos_token_id = -1
    all_special_ids: list = []

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(i) for i in ids)


def _model_and_cache(tokens: int, seed: int):
    from transformers import LlamaForCausalLM

    import common

    torch.manual_seed(seed)
    config = synth.llama_config(SHAPE)
    config.vocab_size = 256
    config.intermediate_size = 256
    model = LlamaForCausalLM(config).to(DEV).float().eval()
    # larger random projections so attention is peaked rather than uniform (logits of order 10)
    with torch.no_grad():
        for layer in model.model.layers:
            layer.self_attn.q_proj.weight.mul_(3.0)
            layer.self_attn.k_proj.weight.mul_(3.0)
    g = torch.Generator("cpu").manual_seed(seed + 1)
    ids = torch.randint(0, config.vocab_size, (1, tokens), generator=g).to(DEV)
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=True)
    keys, values = common.cache_tensors(out.past_key_values)
    return model, [k.clone() for k in keys], [v.clone() for v in values], config


def _checkpoints(keys, values, model):
    """kvtc and progressive calibration dicts with the reference's keys: a full-rank orthonormal
    basis per stream and the mean of the prefill's (de-roped) token vectors."""
    import kvtc

    tokens = keys[0].shape[2]
    cos, sin = kvtc.rope_tables(model, tokens, DEV)
    ctx = synth.make_context(SHAPE, tokens, seed=77)
    ck = synth.kvtc_checkpoint(ctx)
    for kind, tensors in (("key", keys), ("value", values)):
        if kind == "key":
            tensors = [kvtc.derotate(t, cos, sin) for t in tensors]
        matrix = kvtc.token_matrix(tensors)
        ck[kind]["mean"] = matrix.mean(dim=0).cpu()
    return ck, synth.order_checkpoint(SHAPE)


def _answer_both(model, compressed_keys, compressed_values, context, exact, tail, length):
    import common
    from compressed_attention import greedy_answer

    tok = _Tokenizer()
    full = common.build_cache([k.clone() for k in compressed_keys], [v.clone() for v in compressed_values], model)
    with torch.no_grad():
        reply_r, logits_r = greedy_answer(model, tok, None, full, tail, length, max_new_tokens=6, stop_at_eos=False)
        reply_d, logits_d = greedy_answer(model, tok, context, exact, tail, length, max_new_tokens=6,
                                          stop_at_eos=False)
    return reply_r, logits_r, reply_d, logits_d


def _check(logits_r, logits_d, reply_r, reply_d, what):
    diff = float((logits_r - logits_d).abs().max())
    scale = float(logits_r.abs().max())
    print(f"  {what}: max first-step logit diff {diff:.2e} (logit scale {scale:.2e}); replies '{reply_r}' / "
          f"'{reply_d}'", flush=True)
    assert diff <= 1e-2 * scale + 1e-3, f"{what}: logits differ by {diff}"
    assert reply_r == reply_d, f"{what}: replies differ"


def test_prog_direct_matches_rebuilt_and_refine_over_codes():
    import common
    import dimmer
    import methods
    from progressive import question_importance

    print("[case] HF Llama (2 layers) prog@0.3:r0.05 direct vs rebuilt", flush=True)
    model, keys, values, config = _model_and_cache(900, seed=5)
    dimmer.install(model)
    ck, order = _checkpoints(keys, values, model)
    m = methods.Methods("synthetic/llama-3.2", device=DEV, model=model, kvtc=ck, progressive=order)
    compressed = m.apply("prog@0.3:r0.05", keys, values, {})
    stored = compressed.stored
    length = keys[0].shape[2]
    g = torch.Generator("cpu").manual_seed(9)
    tail = torch.randint(0, config.vocab_size, (1, 12), generator=g).to(DEV)
    # question importance over the codes (K4a through the model forward) against the reference's
    # eager question_importance over the FP16 hot cache
    exact = common.build_cache([t.clone() for t in stored.exact["key"]], [t.clone() for t in stored.exact["value"]],
                               model)
    context = stored.context(config.num_attention_heads, exact)
    from progressive import importance_over_codes

    with torch.no_grad():
        imp_codes = importance_over_codes(model, context, exact, tail[0], length).cpu().numpy()
        hot_k, hot_v = stored.hot()
        imp_ref = question_importance(model, hot_k, hot_v, tail[0], length)[stored.start:stored.end].cpu().numpy()
    err = np.abs(imp_codes - imp_ref)
    print(f"  importance over codes vs eager over the hot cache: max err {err.max():.3e} of max "
          f"{np.abs(imp_ref).max():.3e}", flush=True)
    assert (err <= 2e-3 * np.abs(imp_ref).max() + 1e-2 * np.abs(imp_ref)).all(), f"importance err {err.max():.3e}"
    # refine: scored over the codes with a fresh exact cache, top tokens get their cold planes
    exact = common.build_cache([t.clone() for t in stored.exact["key"]], [t.clone() for t in stored.exact["value"]],
                               model)
    packed = stored.stores["key"].packed
    full = packed.tables.pieces
    before = packed.pieces.long().cpu().numpy()
    with torch.no_grad():
        _, _, fetched = compressed.refine(tail[0], length, exact_cache=exact)
    assert fetched > 0
    # the closure selects with dkv_topk (K4b): exactly the top 5 % of the same importance over the codes
    from oracle import scoring_ref

    count = scoring_ref.select_count(0.05, stored.end - stored.start)
    after = packed.pieces.long().cpu().numpy()
    chosen = set(scoring_ref.topk_indices(imp_codes, count).tolist())
    refined = set(np.nonzero((after == full) & (before != full))[0].tolist())
    assert refined == {t for t in chosen if before[t] != full}, "refined tokens are not the top-k of the importance"
    print(f"  refine over the codes: top {count} by dkv_topk, {len(refined)} tokens refined, {fetched} B fetched",
          flush=True)
    hot_k, hot_v = stored.hot()
    exact = common.build_cache([t.clone() for t in stored.exact["key"]], [t.clone() for t in stored.exact["value"]],
                               model)
    context = stored.context(config.num_attention_heads, exact)
    reply_r, logits_r, reply_d, logits_d = _answer_both(model, hot_k, hot_v, context, exact, tail, length)
    _check(logits_r, logits_d, reply_r, reply_d, "prog@0.3:r0.05 after refine")


def test_dkvtc_direct_matches_rebuilt():
    import common
    import dimmer
    import methods
    from compressed_attention import CompressedContext

    print("[case] HF Llama (2 layers) dkvtc@0.3:snap:floor1 direct vs rebuilt", flush=True)
    model, keys, values, config = _model_and_cache(900, seed=6)
    dimmer.install(model)
    ck, _ = _checkpoints(keys, values, model)
    m = methods.Methods("synthetic/llama-3.2", device=DEV, model=model, kvtc=ck)
    length = keys[0].shape[2]
    g = torch.Generator("cpu").manual_seed(10)
    scores = {"snap": [torch.rand(SHAPE.kv_heads, length, generator=g).to(DEV) for _ in range(SHAPE.layers)]}
    compressed = m.apply("dkvtc@0.3:snap:floor1", keys, values, scores)
    context = CompressedContext(m.codec("kvtc"), keys, values, model)
    exact = common.build_cache([l.keys.clone() for l in context.exact_cache.layers],
                               [l.values.clone() for l in context.exact_cache.layers], model)
    tail = torch.randint(0, config.vocab_size, (1, 12), generator=g).to(DEV)
    reply_r, logits_r, reply_d, logits_d = _answer_both(model, compressed.keys, compressed.values, context, exact,
                                                        tail, length)
    _check(logits_r, logits_d, reply_r, reply_d, "dkvtc@0.3:snap:floor1")
