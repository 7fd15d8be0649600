"""The select kernel on constructed score rows (needs an MI355X).

A call fills the workspace; the score rows are then overwritten and the
select stage relaunched alone. The kept channels must be the first F of the
candidates ordered by score (as unsigned float bits, larger first), ties in
ascending candidate order, listed by candidate index. The rows exercise the
radix passes' paths: distinct scores (the cutoff's 24-bit bin holds one key,
so the last pass is skipped), scores sharing their upper 24 bits (the last
pass runs), exact ties at the cutoff and all-equal rows.
"""

import numpy as np
import pytest
import torch

from calibration_free_moe.reader.budget import compile_budget
from calibration_free_moe.reader.progressive import ProgressiveReader, channel_major_down
from tests.synthetic import make_layer

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


def expected_selection(keys: np.ndarray, final_count: int, top_k: int, width: int):
    """Kept mask, next ids (-1 padded), per-slot counts and starts of one row."""
    index = np.arange(keys.size)
    order = np.lexsort((index, -keys.astype(np.int64)))
    kept = np.sort(order[:final_count])
    mask = np.zeros(keys.size, bool)
    mask[kept] = True
    next_ids = np.full(final_count, -1, np.int32)
    next_ids[: kept.size] = kept
    counts = np.array([mask[k * width:(k + 1) * width].sum() for k in range(top_k)], np.int32)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    return mask, next_ids, counts, starts


def score_rows(kind: str, tokens: int, n: int, rng: np.random.Generator) -> np.ndarray:
    if kind == "distinct":
        return rng.random((tokens, n), dtype=np.float32) * 3.0
    if kind == "shared_upper_bits":
        # three 24-bit prefixes, random low bytes: the cutoff's bin is crowded
        upper = 0x3F800000 + 0x100 * rng.integers(0, 3, (tokens, n))
        return (upper | rng.integers(0, 256, (tokens, n))).astype(np.uint32).view(np.float32)
    if kind == "ties":
        return rng.choice(np.array([0.25, 0.5, 1.0, 2.0], np.float32), (tokens, n))
    if kind == "equal":
        return np.full((tokens, n), 0.75, np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("width, top_k, experts", [(256, 4, 8), (1024, 16, 16)])
@pytest.mark.parametrize("kind", ["distinct", "shared_upper_bits", "ties", "equal"])
def test_select_is_the_stable_top_f(width, top_k, experts, kind):
    tokens, hidden = 3, 512
    layer = make_layer(hidden=hidden, width=width, experts=experts, top_k=top_k, rank=16,
                       tokens=tokens, seed=11)
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=top_k,
                          retention=0.123, screen_keep=0.625)
    reader = ProgressiveReader(
        layer.gate_up.to(DEVICE), channel_major_down(layer.down.to(DEVICE)),
        layer.encoder.to(DEVICE), layer.decoder.to(DEVICE), plan, tokens,
        sketch=(layer.codes.to(DEVICE), layer.statistics.to(DEVICE)), selection_score="point",
    )
    hidden_states, ids, weights = (layer.hidden.to(DEVICE), layer.ids.to(DEVICE),
                                   layer.weights.to(DEVICE))
    out = reader(hidden_states, ids, weights)
    n = top_k * width
    rows = score_rows(kind, tokens, n, np.random.default_rng(5))
    reader.scores[0][:tokens].copy_(torch.from_numpy(rows).to(DEVICE))
    reader.launch_stage("select", hidden_states, ids, weights, None, out)
    torch.cuda.synchronize()
    keys = rows.view(np.uint32)
    for t in range(tokens):
        mask, next_ids, counts, starts = expected_selection(keys[t], plan.final_count, top_k, width)
        print(f"select {kind} N={n} token {t}", flush=True)
        assert np.array_equal(reader.selected[t].cpu().numpy().astype(bool), mask)
        assert np.array_equal(reader.candidate_ids[-1][t].cpu().numpy(), next_ids)
        assert np.array_equal(reader.counts[t].cpu().numpy(), counts)
        assert np.array_equal(reader.starts[t].cpu().numpy(), starts)
