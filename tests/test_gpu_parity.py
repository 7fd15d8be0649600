"""HIP reader against the CPU oracle on identical inputs (needs an MI355X).

Every stage is compared bit for bit: routing, rotation, grid values, split
projections, scores, the selected channel ids, exact activations, latents and
the BF16 output. Shapes cover the benchmark configurations (OLMoE, Qwen3-30B-
A3B, the 256-expert I = 512 tail layout) and the reference test suite's edge
cases (padding rows, all-zero inputs, tied experts, full screen, dense bypass,
GELU, Gauss-Hermite scores, HIP-graph replay with changing inputs).
"""

import numpy as np
import pytest
import torch

from calibration_free_moe.reader.budget import compile_budget
from calibration_free_moe.reader.progressive import (
    ProgressiveReader,
    ReaderWorkspace,
    channel_major_down,
)
from oracle import oracle
from tests.synthetic import bits, make_layer, oracle_weights

pytestmark = pytest.mark.gpu

DEVICE = torch.device("cuda:0")


def build(layer, plan, tokens, **options):
    return ProgressiveReader(
        layer.gate_up.to(DEVICE),
        channel_major_down(layer.down.to(DEVICE)),
        layer.encoder.to(DEVICE),
        layer.decoder.to(DEVICE),
        plan,
        tokens,
        sketch=(layer.codes.to(DEVICE), layer.statistics.to(DEVICE)),
        **options,
    )


def run_both(reader, layer, plan, hidden, ids, weights, padding=None, threshold=None):
    out = reader(
        hidden.to(DEVICE), ids.to(DEVICE), weights.to(DEVICE),
        None if padding is None else padding.to(DEVICE),
    )
    torch.cuda.synchronize()
    # token ranges on separate cores (every stage is per token)
    expected = oracle.forward_parallel(
        oracle_weights(layer, reader),
        bits(hidden),
        ids.cpu().numpy(),
        weights.cpu().float().numpy(),
        final_count=plan.final_count,
        keep=plan.screen_coordinates,
        padding=None if padding is None else padding.cpu().numpy().astype(np.uint8),
        point=reader.selection_score == "point",
        gelu=reader.activation == "gelu_tanh",
        threshold=threshold,
    )
    return out, expected


def assert_parity(reader, out, expected, tokens, screened=True):
    t = tokens
    got = {
        "ids": reader.ids[:t].cpu().numpy(),
        "weights": reader.weights[:t].cpu().numpy(),
        "selected": reader.selected[:t].cpu().numpy().astype(np.uint8),
        "next_ids": reader.candidate_ids[-1][:t].cpu().numpy(),
        "counts": reader.counts[:t].cpu().numpy(),
        "starts": reader.starts[:t].cpu().numpy(),
        "tile_starts": reader.tile_starts[:t].cpu().numpy(),
        "activations": bits(reader.activations[:t]),
        "completed": reader.completed[:t].cpu().numpy().astype(np.uint8),
        "partial": reader.partial[:t].cpu().numpy(),
        "out": bits(out),
    }
    if screened:
        got["planes"] = reader.sketch_planes[:t].cpu().numpy()
        got["qvals"] = reader.sketch_values[:t].cpu().numpy()
        got["qexp"] = reader.sketch_exponents[:t].cpu().numpy()
        got["qsums"] = reader.workspace.sketch_sums[:t].cpu().numpy()
        got["scores"] = reader.scores[0][:t].cpu().numpy()
        if reader.plan.screen_coordinates < 128:
            got["coordinates"] = reader.sketch_coordinates[:t].cpu().numpy()
    if reader.rank:
        got["latent"] = reader.latent[:t].cpu().numpy()
    # activations exist only for exactly computed channels; other slots are scratch
    done = expected["completed"].astype(bool)
    got["activations"] = np.where(done, got["activations"], 0)
    expected = dict(expected, activations=np.where(done, expected["activations"], 0))
    if screened:
        # the screen's per-cell sums of the kept grid values
        expected["qsums"] = expected["qvals"].astype(np.int64).sum(-1).astype(np.int32)
    for name, value in got.items():
        want = expected[name]
        if not np.array_equal(value, want):
            mismatch = np.flatnonzero((value != want).reshape(-1))
            raise AssertionError(
                f"{name}: {mismatch.size} of {value.size} differ, first at {mismatch[:5]}"
            )


@pytest.mark.parametrize("tokens", [1, 2, 5])
@pytest.mark.parametrize("score", ["point", "recovery-aware"])
def test_small_layer_bit_exact(tokens, score):
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=40 + tokens)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score=score)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


def test_padding_zero_input_and_gelu():
    tokens = 4
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=44)
    layer.hidden[2] = 0
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.1,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point", activation="gelu_tanh")
    padding = torch.tensor([False, True, False, False])
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights, padding)
    assert_parity(reader, out, expected, tokens)
    assert np.array_equal(expected["next_ids"][2], np.arange(plan.final_count))
    assert not out[1].float().abs().sum()


def test_full_screen_and_bf16_router_weights_int32_ids():
    tokens = 3
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=45)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.2,
                          screen_keep=1.0)
    reader = build(layer, plan, tokens, selection_score="point")
    weights = layer.weights.bfloat16()
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids.int(), weights)
    assert_parity(reader, out, expected, tokens)


def test_dense_bypass():
    tokens = 2
    layer = make_layer(hidden=256, width=64, experts=4, top_k=2, rank=8, tokens=tokens, seed=46)
    plan = compile_budget(hidden_size=256, expert_width=64, top_k=2, retention=1.0)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens, screened=False)


def test_equal_experts_tie_by_expert_id():
    tokens = 2
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=47)
    layer.gate_up[1:4] = layer.gate_up[0]
    layer.down[1:4] = layer.down[0]
    from calibration_free_moe.reader.sketch import block_hadamard_signs, build_sketch
    layer.codes, layer.statistics = build_sketch(layer.gate_up, block_hadamard_signs(512, "cpu"))
    layer.ids[:] = torch.tensor([3, 0, 2, 1])
    layer.weights[:] = 0.25
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
    scores = reader.scores[0][:tokens].reshape(tokens, 4, 256)
    assert torch.equal(scores, scores[:, :1].expand_as(scores))


def test_hot_expert_splits_into_screen_tiles():
    """An expert routed by more than 16 tokens is screened as several tiles of
    at most 16 pairs (one screen workgroup each); results stay bit-exact."""
    tokens, experts, top_k = 40, 8, 4
    layer = make_layer(hidden=512, width=256, experts=experts, top_k=top_k, rank=16,
                       tokens=tokens, seed=61, zipf=1.2)
    layer.ids[:, 0] = 5  # expert 5 in every token: 40 pairs -> tiles of 16, 16, 8
    for t in range(tokens):
        others = [e for e in torch.randperm(experts, generator=torch.Generator().manual_seed(t)).tolist()
                  if e != 5][: top_k - 1]
        layer.ids[t, 1:] = torch.tensor(others)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=top_k, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
    ws = reader.workspace
    total = int(ws.group_total.item())
    tile_experts = ws.group_experts[:total].cpu().tolist()
    starts = ws.group_starts[:total].cpu().tolist()
    counts = ws.group_counts[:total].cpu().tolist()
    pairs = ws.group_pairs[: 16 * total].cpu().tolist()
    pair_tiles = ws.pair_tiles[: tokens * top_k].cpu().tolist()
    masks = ws.tile_masks[: total * 256].cpu().numpy().view(np.uint32).reshape(total, 256)
    assert all(1 <= c <= 16 for c in counts)
    assert tile_experts == sorted(tile_experts)
    assert tile_experts.count(5) == 3 and [c for e, c in zip(tile_experts, counts) if e == 5] == [16, 16, 8]
    assert starts == [16 * z for z in range(total)]
    sorted_ids = expected["ids"]
    selected = expected["selected"].reshape(tokens, top_k, 256).astype(bool)
    seen = []
    for z, (e, first, count) in enumerate(zip(tile_experts, starts, counts)):
        members = pairs[first:first + count]
        assert members == sorted(members)
        assert all(sorted_ids[p // top_k, p % top_k] == e for p in members)
        assert [pair_tiles[p] for p in members] == list(range(first, first + count))
        # bit p of the (tile, channel) mask: pair p of the tile kept the channel
        want = np.zeros(256, np.uint32)
        for position, p in enumerate(members):
            want |= selected[p // top_k, p % top_k].astype(np.uint32) << np.uint32(position)
        assert np.array_equal(masks[z], want)
        seen += members
    assert sorted(seen) == list(range(tokens * top_k))
    # the down kernel's workgroup list: every (token, tile) item once, in the
    # routing's expert order (tiles' pairs, each pair's tiles, then the pairs
    # outside the tiles) cut into eight contiguous runs; entry 8 r + x holds
    # run x's r-th item and the entries past a run hold -1
    max_tiles = ws.down_tiles
    kept = ws.counts[:tokens].cpu().numpy()
    first_tile = ws.down_tile_starts[:tokens].cpu().numpy()
    sequence = []
    def items(p):
        t, k = divmod(p, top_k)
        return [t * max_tiles + int(first_tile[t, k]) + j for j in range(-(-int(kept[t, k]) // 32))]
    for first, count in zip(starts, counts):
        for p in pairs[first:first + count]:
            sequence += items(p)
    for p in range(tokens * top_k):
        if pair_tiles[p] < 0:
            sequence += items(p)
    blocks = -(-tokens * max_tiles // 8) * 8
    order = ws.down_order[:blocks].cpu().numpy().reshape(-1, 8)
    run = -(-len(sequence) // 8)
    for x in range(8):
        want = sequence[x * run:(x + 1) * run]
        assert order[: len(want), x].tolist() == want
        assert (order[len(want):, x] == -1).all()


@pytest.mark.parametrize("score,rank,width", [("point", 16, 256), ("recovery-aware", 16, 256),
                                              ("point", 32, 288), ("recovery-aware", 32, 256)])
def test_grouped_batch_paths_bit_exact(score, rank, width):
    """Batches of 16 or more use the grouped exact rows and per-slot down
    values; padded tokens and a non-local slot exercise their zero results.
    At rank 32 the recovery encoder runs inside the grouped exact launch
    (width 288: a last encoder tile of 32 channels)."""
    tokens, experts, top_k = 24, 16, 4
    layer = make_layer(hidden=512, width=width, experts=experts, top_k=top_k, rank=rank,
                       tokens=tokens, seed=71)
    layer.ids[5, 2] = 99  # no local expert: reads nothing, contributes zero
    padding = torch.zeros(tokens, dtype=torch.bool)
    padding[[3, 10]] = True
    plan = compile_budget(hidden_size=512, expert_width=width, top_k=top_k, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score=score)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights, padding)
    assert_parity(reader, out, expected, tokens)


def test_grouped_batch_qwen3_shape_bit_exact():
    tokens = 32
    layer = make_layer(hidden=2048, width=768, experts=128, top_k=8, rank=32, tokens=tokens,
                       seed=72)
    plan = compile_budget(hidden_size=2048, expert_width=768, top_k=8, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


def test_threshold_selection():
    tokens = 3
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=48)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    probe = build(layer, plan, tokens, selection_score="point")
    probe(layer.hidden.to(DEVICE), layer.ids.to(DEVICE), layer.weights.to(DEVICE))
    tau = float(probe.scores[0][0].sort(descending=True).values[60])
    reader = build(layer, plan, tokens, selection_score="point", selection_threshold=tau)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights,
                             threshold=tau)
    assert_parity(reader, out, expected, tokens)
    assert reader.report()["charged_bytes"] > 0


@pytest.mark.parametrize(
    "hidden,width,experts,top_k,retention,tokens",
    [
        (2048, 1024, 64, 8, 0.123, 1),  # OLMoE-1B-7B layer, batch one
        (2048, 768, 128, 8, 0.123, 1),  # Qwen3-30B-A3B layer, batch one
        (2048, 768, 128, 8, 0.123, 4),
        (2048, 512, 256, 8, 0.123, 2),  # 256 experts, I = 512 block-paired tails
    ],
)
def test_benchmark_shapes_bit_exact(hidden, width, experts, top_k, retention, tokens):
    layer = make_layer(hidden=hidden, width=width, experts=experts, top_k=top_k, rank=32,
                       tokens=tokens, seed=50 + tokens)
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=top_k,
                          retention=retention, screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
    report = reader.report()
    charged = (plan.selected_weight_bytes() + plan.recovery_read_bytes(32)
               + plan.selection_read_bytes(False) + plan.sketch_read_bytes(False) + hidden)
    assert report["charged_bytes"] == tokens * charged
    assert report["reference_bytes"] == tokens * plan.native_read_bytes()


@pytest.mark.parametrize(
    "hidden,width,activation,tokens,keep,score,retention",
    [
        # H = 2816 (22 blocks): seven three-block screen splits and a last one of one block
        (2816, 704, "gelu_tanh", 1, 0.625, "point", 0.125),
        (2816, 704, "gelu_tanh", 1, 1.0, "recovery-aware", 0.2),
        (2816, 704, "gelu_tanh", 5, 0.625, "point", 0.125),
        (2816, 512, "silu", 16, 1.0, "recovery-aware", 0.1),
        # H = 4096 (32 blocks): four-block splits, eight 16-byte hidden parts per lane
        (4096, 512, "silu", 1, 0.625, "recovery-aware", 0.123),
        (4096, 512, "silu", 20, 0.625, "point", 0.123),
        # expert widths past 1024: Qwen3-235B's 1536 (24 encoder tiles), and 2048
        (4096, 1536, "silu", 1, 0.625, "point", 0.123),
        (2048, 1536, "silu", 18, 0.625, "recovery-aware", 0.123),
        (2048, 2048, "silu", 5, 0.625, "point", 0.06),
    ],
    ids=["gemma-t1-keep80", "gemma-t1-dense-gh5", "gemma-t5", "gemma-grouped-gh5",
         "h4096-t1-gh5", "h4096-grouped", "qwen235b-t1", "i1536-grouped-gh5", "i2048-t5"],
)
def test_wide_layers_bit_exact(hidden, width, activation, tokens, keep, score, retention):
    """Hidden sizes above 2048 (Gemma 4's 2816, and 4096) run the span-4 screens
    and the eight-part exact rows, and widths above 1024 fold more than 16
    encoder tiles; every stage stays bit-exact against the oracle, at batch 1
    (per-channel-tile screen), 5 (fused screen, per-token exact rows) and from
    16 (grouped rows and down order)."""
    layer = make_layer(hidden=hidden, width=width, experts=4, top_k=2, rank=32, tokens=tokens,
                       seed=hidden + width + tokens)
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=2, retention=retention,
                          screen_keep=keep)
    reader = build(layer, plan, tokens, activation=activation, selection_score=score)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


@pytest.mark.parametrize(
    "hidden,width,tokens,score",
    [
        # B = 9 blocks: eight splits of two blocks, the last three hold none
        (1152, 256, 1, "point"),
        (1152, 256, 5, "point"),
        (1152, 256, 17, "recovery-aware"),
        # B = 18: span 3 (the wide screens), splits 6 and 7 hold none
        (2304, 512, 1, "recovery-aware"),
        (2304, 512, 20, "point"),
    ],
    ids=["h1152-t1", "h1152-t5", "h1152-grouped-gh5", "h2304-t1-gh5", "h2304-grouped"],
)
def test_screen_splits_past_the_blocks_bit_exact(hidden, width, tokens, score):
    """With B = 9 or 18 blocks the eight screen splits of ceil(B / 8) blocks
    end before the last split: the empty splits add a zero partial (the
    oracle's estimate + 0.0), in every screen kernel."""
    layer = make_layer(hidden=hidden, width=width, experts=6, top_k=2, rank=32, tokens=tokens,
                       seed=hidden + tokens)
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=2, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score=score)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


def test_routing_of_more_pairs_than_one_batch_per_thread():
    """3072 experts and 4096 routed pairs: the experts' LDS lists keep the
    routing block at 256 threads, so each thread routes 16 pairs, the first 8
    from one round trip and the rest in further ones; padded tokens mixed in."""
    tokens = 256
    layer = make_layer(hidden=256, width=64, experts=3072, top_k=16, rank=8, tokens=tokens, seed=5)
    plan = compile_budget(hidden_size=256, expert_width=64, top_k=16, retention=0.2, screen_keep=0.625)
    padding = torch.zeros(tokens, dtype=torch.bool)
    padding[::7] = True
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights, padding)
    assert_parity(reader, out, expected, tokens)


def test_graph_replay_with_changing_inputs():
    tokens = 4
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=60)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    x = layer.hidden.to(DEVICE).clone()
    ids = layer.ids.to(DEVICE).clone()
    weights = layer.weights.to(DEVICE).clone()
    padding = torch.zeros(tokens, dtype=torch.bool, device=DEVICE)
    out = reader(x, ids, weights, padding)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = reader(x, ids, weights, padding)
    generator = torch.Generator().manual_seed(3)
    for replay in range(4):
        x.copy_(torch.randn(tokens, 512, generator=generator).bfloat16())
        if replay == 2:
            x.zero_()
        padding.zero_()
        padding[1] = replay % 2 == 1
        ids.copy_(ids.flip(1))
        weights.uniform_(0.2, 0.8)
        reader.read_work.zero_()
        graph.replay()
        torch.cuda.synchronize()
        expected = oracle.forward(
            oracle_weights(layer, reader), bits(x), ids.cpu().numpy(),
            weights.cpu().numpy(), final_count=plan.final_count, keep=80,
            padding=padding.cpu().numpy().astype(np.uint8),
        )
        assert_parity(reader, out, expected, tokens)
        active = int((~padding).sum())
        assert reader.report()["reference_bytes"] == active * plan.native_read_bytes()


def test_shared_workspace_between_layers():
    tokens = 3
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    small = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.08,
                           screen_keep=0.625)
    first = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=61)
    second = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens, seed=62)
    workspace = ReaderWorkspace(plan, 8, 16, tokens, DEVICE)
    a = build(first, plan, tokens, selection_score="point", workspace=workspace)
    b = build(second, small, tokens, selection_score="point", workspace=workspace)
    assert a.workspace_bytes > 0 and b.workspace_bytes == 0
    out_b, expected_b = run_both(b, second, small, second.hidden, second.ids, second.weights)
    assert_parity(b, out_b, expected_b, tokens)
    out_a, expected_a = run_both(a, first, plan, first.hidden, first.ids, first.weights)
    assert_parity(a, out_a, expected_a, tokens)


def test_large_batch_selection_is_top_f_of_own_scores():
    """Batch 64 at the OLMoE shape: size-independent properties plus sampled parity."""
    tokens = 64
    layer = make_layer(hidden=2048, width=1024, experts=64, top_k=8, rank=32, tokens=tokens,
                       seed=70)
    plan = compile_budget(hidden_size=2048, expert_width=1024, top_k=8, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
    scores = reader.scores[0][:tokens].cpu()
    order = scores.argsort(dim=1, descending=True, stable=True)[:, : plan.final_count]
    membership = torch.zeros_like(scores, dtype=torch.bool).scatter_(1, order, True)
    assert torch.equal(reader.selected[:tokens].cpu(), membership)


@pytest.fixture(scope="module")
def skewed_qwen3_layer():
    """C4: the Qwen3-30B-A3B shape at batch 256 with Zipf(1.2) expert popularity."""
    return make_layer(hidden=2048, width=768, experts=128, top_k=8, rank=32, tokens=256,
                      seed=80, zipf=1.2, device=DEVICE)


@pytest.mark.parametrize("retention", [0.06, 0.123, 0.25])
def test_skewed_routing_qwen3_batch_256(skewed_qwen3_layer, retention):
    """Load-imbalanced routing (the hottest expert serves most tokens, many
    experts none) over the retention sweep F = 369 / 756 / 1536: hot experts
    split into many 16-pair tiles, cold ones hold one pair."""
    layer = skewed_qwen3_layer
    tokens = 256
    counts = torch.bincount(layer.ids.reshape(-1).cpu(), minlength=128)
    assert counts.max() > 64  # the hottest expert alone needs five or more tiles
    plan = compile_budget(hidden_size=2048, expert_width=768, top_k=8, retention=retention,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
    # the grouping under skew: experts ascending, each expert's pairs in pair
    # order cut into tiles of 16, every pair in exactly one tile slot
    ws = reader.workspace
    total = int(ws.group_total.item())
    tile_experts = ws.group_experts[:total].cpu().numpy()
    tile_counts = ws.group_counts[:total].cpu().numpy()
    slots = ws.group_pairs[: 16 * total].cpu().numpy().reshape(total, 16)
    pair_tiles = ws.pair_tiles[: tokens * 8].cpu().numpy()
    sorted_ids = expected["ids"].reshape(-1)
    assert (np.diff(tile_experts) >= 0).all()
    order = np.concatenate([slots[z, : tile_counts[z]] for z in range(total)])
    assert np.array_equal(np.sort(order), np.arange(tokens * 8))
    for expert in np.unique(tile_experts):
        members = np.concatenate([slots[z, : tile_counts[z]] for z in np.flatnonzero(tile_experts == expert)])
        assert np.array_equal(members, np.flatnonzero(sorted_ids == expert))
        assert (tile_counts[tile_experts == expert][:-1] == 16).all()
    for z in range(total):
        assert np.array_equal(pair_tiles[slots[z, : tile_counts[z]]], 16 * z + np.arange(tile_counts[z]))


@pytest.fixture(scope="module")
def fine_grained_layer():
    """C5: 256 experts of width 512 (block-paired sketch tails) at batch 128."""
    return make_layer(hidden=2048, width=512, experts=256, top_k=8, rank=32, tokens=128,
                      seed=90, device=DEVICE)


@pytest.mark.parametrize("keep", [1.0, 0.625])
def test_fine_grained_experts_batch_128(fine_grained_layer, keep):
    """Point-only screening over every coordinate (keep 1.0) against the
    two-stage screen that keeps 80 of 128 rotated coordinates per block."""
    layer = fine_grained_layer
    tokens = 128
    plan = compile_budget(hidden_size=2048, expert_width=512, top_k=8, retention=0.123,
                          screen_keep=keep)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)
