"""Seeded sweep of layer shapes and call options, each bit-exact to the oracle
(needs an MI355X).

Every case draws its shape (H, I, E, K, rank), batch, plan (retention, screen
keep), score, activation, router formats, skew and padding from its own seed, so the
sweep crosses the per-token and grouped paths, the small and fused screens,
both hidden-part widths' neighbours, encoder tiles with tails, equal-expert
ties and padded rows in combinations the targeted tests do not name. Every
stage's output is compared bit for bit (`assert_parity`).
"""

import numpy as np
import pytest
import torch

from calibration_free_moe.reader.budget import compile_budget
from tests.synthetic import make_layer, make_routed_layer
from tests.test_gpu_parity import DEVICE, assert_parity, build, run_both

pytestmark = pytest.mark.gpu

CASES = 96


def draw(case: int) -> dict:
    """The case's configuration (a pure function of its index)."""
    rng = np.random.default_rng(9000 + case)
    experts = int(rng.choice([2, 3, 5, 8, 13, 24, 40, 64]))
    top_k = int(rng.integers(1, min(8, experts) + 1))
    tokens = int(rng.choice([1, 2, 3, 7, 15, 16, 17, 24, 33, 64, 100]))
    return {
        "hidden": int(rng.choice([256, 384, 512, 640, 1152, 2048, 2816])),
        "width": int(rng.choice([64, 128, 192, 256, 288, 320, 512])),
        "experts": experts,
        "top_k": top_k,
        "rank": int(rng.choice([8, 16, 32])),
        "tokens": tokens,
        "retention": float(rng.choice([0.06, 0.123, 0.25, 0.5])),
        "keep": float(rng.choice([0.625, 1.0])),
        "score": str(rng.choice(["point", "recovery-aware"])),
        "activation": str(rng.choice(["silu", "gelu_tanh"])),
        "ids64": bool(rng.integers(2)),
        "weights16": bool(rng.integers(2)),
        "padded": [bool(p) for p in rng.random(tokens) < 0.2],
        "tie": bool(rng.random() < 0.25) and top_k > 1,
        "zipf": float(rng.choice([1.2, 2.0])) if rng.random() < 0.25 else None,
    }


@pytest.mark.parametrize("case", range(CASES))
def test_random_configuration_bit_exact(case):
    c = draw(case)
    print(f"case {case}: {c}", flush=True)
    tokens = c["tokens"]
    layer = make_layer(hidden=c["hidden"], width=c["width"], experts=c["experts"],
                       top_k=c["top_k"], rank=c["rank"], tokens=tokens, seed=700 + case,
                       zipf=c["zipf"])
    ids = layer.ids.clone()
    if c["tie"]:
        ids[0, 1] = ids[0, 0]  # a token naming one expert twice
    plan = compile_budget(hidden_size=c["hidden"], expert_width=c["width"], top_k=c["top_k"],
                          retention=c["retention"], screen_keep=c["keep"])
    reader = build(layer, plan, tokens, selection_score=c["score"], activation=c["activation"])
    ids = ids if c["ids64"] else ids.int()
    weights = layer.weights.bfloat16() if c["weights16"] else layer.weights
    padding = torch.tensor(c["padded"]) if any(c["padded"]) else None
    out, expected = run_both(reader, layer, plan, layer.hidden, ids, weights, padding)
    screened = plan.final_count < plan.candidate_count
    assert_parity(reader, out, expected, tokens, screened=screened)
    if padding is not None:
        assert not out[padding.to(out.device)].float().abs().sum()


WIDE_CASES = 24


def draw_wide(case: int) -> dict:
    """A wide-layer case: the benchmark-scale shapes, skewed sizes and modes."""
    rng = np.random.default_rng(19000 + case)
    hidden = int(rng.choice([2048, 2816, 4096]))
    width = int(rng.choice([512, 768, 1024, 1536, 2048]))
    top_k = int(rng.choice([4, 6, 8, 10, 16]))
    while top_k * width > 16384:
        top_k //= 2
    experts = int(rng.choice([16, 64, 128, 256]))
    while experts > top_k and experts * 2 * width * hidden > 1.0e8:
        experts //= 2
    experts = max(experts, top_k)
    tokens = int(rng.choice([1, 4, 16, 48, 128]))
    while tokens * top_k > 8192:
        tokens //= 2
    mode = str(rng.choice(["top", "top", "top", "top", "threshold", "dense"]))
    return {
        "hidden": hidden, "width": width, "experts": experts, "top_k": top_k,
        "rank": int(rng.choice([16, 32, 64])), "tokens": tokens, "mode": mode,
        "retention": 1.0 if mode == "dense" else float(rng.choice([0.06, 0.123, 0.25])),
        "keep": 1.0 if mode == "dense" else float(rng.choice([0.625, 1.0])),
        "score": str(rng.choice(["point", "recovery-aware"])) if mode != "threshold" else "point",
        "padded": [bool(p) for p in rng.random(tokens) < 0.1],
    }


@pytest.mark.parametrize("case", range(WIDE_CASES))
def test_random_wide_configuration_bit_exact(case):
    c = draw_wide(case)
    print(f"wide case {case}: {c}", flush=True)
    tokens = c["tokens"]
    layer = make_routed_layer(hidden=c["hidden"], width=c["width"], experts=c["experts"],
                              top_k=c["top_k"], rank=c["rank"], tokens=tokens, seed=900 + case)
    plan = compile_budget(hidden_size=c["hidden"], expert_width=c["width"], top_k=c["top_k"],
                          retention=c["retention"], screen_keep=c["keep"])
    padding = torch.tensor(c["padded"]) if any(c["padded"]) else None
    threshold = None
    if c["mode"] == "threshold":
        # a threshold that keeps about a tenth of the first token's candidates
        probe = build(layer, plan, tokens, selection_score="point")
        probe(layer.hidden.to(DEVICE), layer.ids.to(DEVICE), layer.weights.to(DEVICE))
        ranked = probe.scores[0][0].sort(descending=True).values
        threshold = float(ranked[plan.candidate_count // 10])
        del probe
    reader = build(layer, plan, tokens, selection_score=c["score"],
                   selection_threshold=threshold)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights, padding,
                             threshold=threshold)
    assert_parity(reader, out, expected, tokens, screened=c["mode"] != "dense")
