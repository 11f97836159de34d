"""Seeded synthetic Llama-3.2-shaped compressed caches (no model download is possible offline).

Stands in for the reference's calibration artefacts (scripts/fit_kvtc.py,
scripts/fit_progressive.py) and prefill caches:

* Key and value bases: orthonormal ``[F, r]`` (Q of a QR of a seeded Gaussian),
  F = layers * kv_heads * head_dim, row f = (layer * kv_heads + head) * head_dim + d,
  exactly the feature order of scripts/kvtc.py:50-52 (``token_matrix``).
* PCA spectrum lambda_i = i^-1.5; coefficients sqrt(lambda_i) * N(0, 1).
* Means: N(0, mean_scale^2) per feature.
* Per-token precision: 0 planes with probability ``zero_frac``, else
  ``floor + min(Geometric(p), 8 - floor)`` planes, with p chosen so the hot
  tier meets a byte budget when one is given (then trimmed to fit exactly).
* Progressive order: plane-major (every group's plane 0, then plane 1, ...),
  so a token with m planes keeps ``m * G`` pieces.
* Exact tokens (sinks, recent window, new tokens): decoded from
  full-precision coefficients, keys RoPE'd at their positions.

Everything is generated with ``torch.Generator('cpu')`` seeds so CPU tests
and GPU runs see the same numbers.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

PLANES = 8
HEADER_BYTES = 4
PIECE_BYTES = 8


@dataclass(frozen=True)
class ModelShape:
    layers: int
    kv_heads: int
    head_dim: int
    q_heads: int
    rank: int
    rope_theta: float = 500000.0

    @property
    def features(self) -> int:
        return self.layers * self.kv_heads * self.head_dim

    @property
    def groups(self) -> int:
        return self.rank // 64

    @property
    def gqa(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def exact_bytes(self) -> int:
        """FP16 bytes of one token's keys (or values), scripts/kvtc.py:133-134."""
        return self.features * 2


SHAPE_1B = ModelShape(layers=16, kv_heads=8, head_dim=64, q_heads=32, rank=1024)
SHAPE_3B = ModelShape(layers=28, kv_heads=8, head_dim=128, q_heads=24, rank=2048)


def llama_config(shape: ModelShape):
    """A local LlamaConfig with Llama-3.2's llama3 RoPE parameters (constructing it fetches nothing)."""
    from transformers import LlamaConfig

    return LlamaConfig(
        hidden_size=shape.head_dim * shape.q_heads, num_attention_heads=shape.q_heads,
        num_key_value_heads=shape.kv_heads, head_dim=shape.head_dim, num_hidden_layers=shape.layers,
        max_position_embeddings=131072, intermediate_size=64, vocab_size=128,
        rope_parameters={"rope_type": "llama3", "rope_theta": shape.rope_theta, "factor": 32.0,
                         "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                         "original_max_position_embeddings": 8192})


def rope_tables(shape: ModelShape, tokens: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin float32 [tokens, head_dim] for positions 0..tokens-1 via transformers'
    LlamaRotaryEmbedding, the call scripts/kvtc.py:32-37 makes through the model."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    emb = LlamaRotaryEmbedding(llama_config(shape)).to(device)
    positions = torch.arange(tokens, device=device)[None]
    cos, sin = emb(torch.zeros(1, device=device, dtype=torch.float32), positions)
    return cos[0].float().contiguous(), sin[0].float().contiguous()


def _gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def orthonormal_basis(features: int, rank: int, seed: int, device="cpu") -> torch.Tensor:
    """Q of a QR of a seeded Gaussian [features, rank], as float32.  The QR runs on the host
    (float64 for small bases, float32 for model-sized ones) so every device sees the same basis."""
    g = _gen(seed)
    a = torch.randn(features, rank, generator=g, dtype=torch.float32)
    q, _ = torch.linalg.qr(a.double() if features * rank <= (1 << 23) else a)
    return q.float().to(device).contiguous()


def eigen_scale(rank: int) -> torch.Tensor:
    return torch.arange(1, rank + 1, dtype=torch.float64).pow(-0.75).float()


def coefficients(n: int, rank: int, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(seed)
    return (torch.randn(n, rank, generator=g, dtype=torch.float32) * eigen_scale(rank)).to(device)


def stream_bytes(planes: np.ndarray, groups: int) -> np.ndarray:
    """Hot bytes of tokens whose every group keeps ``planes`` planes (plane-major order)."""
    planes = np.asarray(planes)
    return np.where(planes > 0, groups * (HEADER_BYTES + PIECE_BYTES * planes), 0)


def _expected_planes(p: float, floor: int, zero_frac: float) -> float:
    q = 1.0 - p
    cap = PLANES - floor
    extra = q * (1 - q**cap) / p if p < 1 else 0.0
    return (1 - zero_frac) * (floor + extra)


def plane_counts(n: int, groups: int, seed: int, zero_frac: float = 0.05, floor: int = 2, p: float | None = None,
                 stream_budget: float | None = None) -> np.ndarray:
    """Per-token plane counts (int64 [n], 0 or floor..8).

    With ``stream_budget`` (average hot bytes per token of this stream), p is
    solved so the expected size meets it, then random tokens above the floor
    lose planes until the total fits."""
    if p is None:
        if stream_budget is None:
            p = 0.5
        else:
            target_planes = (stream_budget / groups - HEADER_BYTES * (1 - zero_frac)) / PIECE_BYTES
            lo, hi = 1e-4, 1.0
            for _ in range(60):
                mid = 0.5 * (lo + hi)
                if _expected_planes(mid, floor, zero_frac) > target_planes:
                    lo = mid
                else:
                    hi = mid
            p = hi
    rng = np.random.default_rng(seed)
    extra = np.minimum(rng.geometric(p, size=n) - 1, PLANES - floor)
    planes = floor + extra
    planes[rng.random(n) < zero_frac] = 0
    if stream_budget is not None:
        limit = int(stream_budget * n)
        total = int(stream_bytes(planes, groups).sum())
        order = rng.permutation(n)
        i = 0
        while total > limit:
            t = order[i % n]
            i += 1
            if planes[t] > floor:
                planes[t] -= 1
                total -= PIECE_BYTES * groups
            if i > 16 * n:
                raise ValueError("budget below the plane floor")
    return planes.astype(np.int64)


@dataclass
class SyntheticContext:
    """A compressed conversation: bases, means, middle-token coefficients and plane maps, exact tokens."""

    shape: ModelShape
    tokens: int
    sinks: int
    recent: int
    basis: dict
    mean: dict
    coef: dict          # middle tokens, float32 [middle, rank]
    planes: dict        # int64 [middle]
    exact_coef: dict    # float32 [E_ctx, rank] for sinks + recent
    seed: int
    extra: dict = field(default_factory=dict)

    @property
    def start(self) -> int:
        return min(self.sinks, self.tokens)

    @property
    def end(self) -> int:
        return max(self.start, self.tokens - self.recent)

    @property
    def middle(self) -> int:
        return self.end - self.start

    def exact_positions(self) -> torch.Tensor:
        return torch.cat([torch.arange(0, self.start), torch.arange(self.end, self.tokens)])

    def pieces(self, kind: str) -> np.ndarray:
        return self.planes[kind] * self.shape.groups


def budget_per_stream(shape: ModelShape, tokens: int, sinks: int, recent: int, budget: float) -> float:
    """Average hot bytes per middle token per stream left by a budget (scripts/progressive.py:141-142,166),
    after the exact tokens and the 1-byte rung id."""
    start = min(sinks, tokens)
    end = max(start, tokens - recent)
    middle = end - start
    budget_bytes = int(budget * tokens * 2 * shape.exact_bytes)
    remaining = budget_bytes - (tokens - middle) * 2 * shape.exact_bytes
    return remaining / (2 * middle) - 1


def make_context(shape: ModelShape, tokens: int, seed: int, sinks: int = 4, recent: int = 32,
                 budget: float | None = None, zero_frac: float = 0.05, floor: int = 2, p: float | None = None,
                 mean_scale: float = 0.01, device="cpu", basis=None, mean=None,
                 budget_over_middle: bool = False, budget_shape: ModelShape | None = None) -> SyntheticContext:
    """``basis`` / ``mean`` (dicts by stream) let several conversations share one model's tables.
    ``budget_over_middle`` applies ``budget`` to the compressed tokens alone (budget x FP16 bytes per
    compressed token) instead of the whole conversation with its exact tokens.  ``budget_shape`` is
    the model whose FP16 bytes the budget is a fraction of (default ``shape``): a few-layer slice of a
    model then gets the plane maps the whole model's budget gives."""
    middle = max(0, tokens - min(sinks, tokens) - recent)
    stream_budget = None
    if budget is not None:
        bshape = budget_shape or shape
        stream_budget = (budget * bshape.exact_bytes - 1 if budget_over_middle
                         else budget_per_stream(bshape, tokens, sinks, recent, budget))
    if basis is None:
        basis = {"key": orthonormal_basis(shape.features, shape.rank, seed + 1, device),
                 "value": orthonormal_basis(shape.features, shape.rank, seed + 2, device)}
    if mean is None:
        g = _gen(seed + 3)
        mean = {kind: (torch.randn(shape.features, generator=g) * mean_scale).to(device) for kind in ("key", "value")}
    coef = {"key": coefficients(middle, shape.rank, seed + 4, device),
            "value": coefficients(middle, shape.rank, seed + 5, device)}
    planes = {"key": plane_counts(middle, shape.groups, seed + 6, zero_frac, floor, p, stream_budget),
              "value": plane_counts(middle, shape.groups, seed + 7, zero_frac, floor, p, stream_budget)}
    n_exact = tokens - middle
    exact_coef = {"key": coefficients(n_exact, shape.rank, seed + 8, device),
                  "value": coefficients(n_exact, shape.rank, seed + 9, device)}
    return SyntheticContext(shape, tokens, sinks, recent, basis, mean, coef, planes, exact_coef, seed)


def decode_exact(ctx: SyntheticContext, coef: dict, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Full-precision decode of exact tokens -> per-layer keys/values float32 [L, Hkv, E, d], keys RoPE'd."""
    s = ctx.shape
    out = {}
    for kind in ("key", "value"):
        x = coef[kind] @ ctx.basis[kind].T + ctx.mean[kind]  # [E, F]
        x = x.view(-1, s.layers, s.kv_heads, s.head_dim).permute(1, 2, 0, 3).contiguous()  # [L, Hkv, E, d]
        if kind == "key":
            c, sn = cos[positions], sin[positions]
            half = s.head_dim // 2
            rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
            x = x * c + rot * sn
        out[kind] = x.contiguous()
    return out["key"], out["value"]


def make_queries(shape: ModelShape, q_len: int, seed: int, device="cpu", dtype=torch.float32,
                 scale: float = 1.0, layers: int | None = None) -> torch.Tensor:
    """Query tokens [L, 1, Hq, q_len, d] ~ N(0, scale^2) (RoPE already applied, as HF passes them)."""
    g = _gen(seed)
    layers = shape.layers if layers is None else layers
    q = torch.randn(layers, 1, shape.q_heads, q_len, shape.head_dim, generator=g) * scale
    return q.to(dtype).to(device)


def causal_mask(q_len: int, exact_ctx: int, device="cpu") -> torch.Tensor:
    """Additive mask [1, 1, q_len, exact_ctx + q_len]: context exact tokens visible, new tokens causal."""
    m = torch.zeros(q_len, exact_ctx + q_len)
    m[:, exact_ctx:] = torch.triu(torch.full((q_len, q_len), float("-inf")), diagonal=1)
    return m[None, None].to(device)


def ragged_lengths(count: int, lo: int, hi: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=count)]


def stream_budget_bytes(shape: ModelShape, budget: float) -> float:
    """Per-stream hot bytes per token for a fraction of FP16 (no exact tokens)."""
    return budget * shape.exact_bytes


class RopeModel(torch.nn.Module):
    """The one part of a Llama model the codecs call: ``model.model.rotary_emb`` and ``config``
    (scripts/kvtc.py:32-37).  Built from the local config; no weights."""

    def __init__(self, shape: ModelShape, device="cpu"):
        super().__init__()
        from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

        self.config = llama_config(shape)
        self.model = torch.nn.Module()
        self.model.rotary_emb = LlamaRotaryEmbedding(self.config).to(device)


def ladder_rungs(groups: int) -> torch.Tensor:
    """kvtc bit-width ladder [rungs, groups] over {0, 2, 4, 8}, coarse -> fine: rung r gives the
    leading groups more bits (the shape scripts/fit_kvtc.py produces from calibration)."""
    rows = []
    for r in range(1, 9):
        bits = torch.zeros(groups, dtype=torch.long)
        n8 = (groups * r) // 16
        n4 = min(groups - n8, (groups * r) // 8)
        n2 = min(groups - n8 - n4, (groups * r) // 4)
        bits[:n8] = 8
        bits[n8:n8 + n4] = 4
        bits[n8 + n4:n8 + n4 + n2] = 2
        rows.append(bits)
    return torch.stack(rows)


def kvtc_checkpoint(ctx: "SyntheticContext", model_id: str = "synthetic/llama-3.2", group: int = 64) -> dict:
    """A kvtc calibration dict with the keys scripts/kvtc.py:108-131 reads, from a synthetic context."""
    s = ctx.shape
    rungs = ladder_rungs(s.rank // group)
    saved = {"model": model_id, "layers": s.layers, "heads": s.kv_heads, "head_dim": s.head_dim, "group": group,
             "sinks": ctx.sinks}
    for kind in ("key", "value"):
        sizes = [int((b.float() * group / 8).sum() + 4 * (b > 0).sum()) for b in rungs]
        saved[kind] = {"mean": ctx.mean[kind].float().cpu(), "basis": ctx.basis[kind].float().cpu(), "rungs": rungs,
                       "rung_bytes": sizes}
    return saved


def order_checkpoint(shape: ModelShape, model_id: str = "synthetic/llama-3.2") -> dict:
    """A progressive-order dict with the keys scripts/progressive.py:124-129 reads: plane-major order."""
    groups = shape.groups
    sizes, planes, level = [0.0], [[0] * groups], [0] * groups
    for k in range(PLANES * groups):
        g = k % groups
        sizes.append(sizes[-1] + PIECE_BYTES + (HEADER_BYTES if level[g] == 0 else 0))
        level[g] += 1
        planes.append(list(level))
    entry = {"planes": torch.tensor(planes, dtype=torch.uint8), "prefix_bytes": torch.tensor(sizes, dtype=torch.float64),
             "rungs": [groups * m for m in range(1, PLANES + 1)]}
    return {"model": model_id, "key": dict(entry), "value": dict(entry)}


def prefill_cache(ctx: "SyntheticContext", coef_middle: dict | None = None, device="cpu", dtype=torch.float16,
                  compute_device="cpu"):
    """Per-layer keys/values [1, Hkv, T, d] of a whole conversation (sinks, middle, recent), keys RoPE'd:
    what a prefill leaves in a DynamicCache (scripts/common.py:62-67).  ``compute_device`` is where
    the float32 decode runs (the context's tensors must live there)."""
    s = ctx.shape
    coef_middle = ctx.coef if coef_middle is None else coef_middle
    cos, sin = rope_tables(s, ctx.tokens, compute_device)
    coef = {kind: torch.cat([ctx.exact_coef[kind][:ctx.start].to(compute_device), coef_middle[kind].to(compute_device),
                             ctx.exact_coef[kind][ctx.start:].to(compute_device)]) for kind in ("key", "value")}
    keys, values = decode_exact(ctx, coef, torch.arange(ctx.tokens, device=compute_device), cos, sin)
    return ([keys[l][None].to(device=device, dtype=dtype) for l in range(s.layers)],
            [values[l][None].to(device=device, dtype=dtype) for l in range(s.layers)])


__all__ = ["ModelShape", "SHAPE_1B", "SHAPE_3B", "SyntheticContext", "make_context", "make_queries", "rope_tables",
           "decode_exact", "plane_counts", "orthonormal_basis", "coefficients", "causal_mask", "ragged_lengths",
           "budget_per_stream", "stream_bytes", "llama_config", "RopeModel",
           "ladder_rungs", "kvtc_checkpoint", "order_checkpoint", "prefill_cache"]
