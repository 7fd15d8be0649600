"""Operator paths the runtime reaches besides a plain call (needs an MI355X).

* Early rotation: `prepare_input(hidden, padding)` then
  `reader(..., input_prepared=True)`, the order the reference's vLLM binding
  uses (runtime/experts.py:402-427, :497-505; progressive.py:3829-3873).
* The default constructor, which builds the sketch itself (`sketch=None`).
* Select and exact in one launch (up to four tokens) against the stages
  relaunched one at a time, which run the separate kernels.
* The configurations without a test elsewhere: Qwen3-30B-A3B at batch 128 and
  the 256-expert layer at batch 1, with point-only (keep 1.0) and two-stage
  (keep 0.625) screening.

Every case is held bit for bit to the CPU oracle on the reader's own tensors.
"""

import numpy as np
import pytest
import torch

from calibration_free_moe.reader import _ext
from calibration_free_moe.reader.budget import compile_budget
from calibration_free_moe.reader.progressive import ProgressiveReader, channel_major_down
from tests.synthetic import make_layer
from tests.test_gpu_parity import DEVICE, assert_parity, build, run_both

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens", [1, 24])
def test_prepared_input_equals_a_plain_call(tokens):
    """The prepared call reads the rotation that prepare_input left; a stale
    rotation from an earlier call with other rows would change the result."""
    layer = make_layer(hidden=512, width=256, experts=16, top_k=4, rank=16, tokens=tokens,
                       seed=100 + tokens)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    hidden = layer.hidden.to(DEVICE)
    ids, weights = layer.ids.to(DEVICE), layer.weights.to(DEVICE)
    padding = torch.zeros(tokens, dtype=torch.bool, device=DEVICE)
    padding[-1] = True
    if tokens > 2:
        padding[tokens // 3] = True
    plain = reader(hidden, ids, weights, padding).clone()
    torch.cuda.synchronize()
    # leave another batch's rotation in the workspace
    other = torch.randn(tokens, 512, generator=torch.Generator().manual_seed(7)).bfloat16()
    reader(other.to(DEVICE), ids, weights)
    assert reader.prepare_input(hidden, padding) is True
    out = reader(hidden, ids, weights, padding, input_prepared=True)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    _, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights,
                           padding.cpu())
    # run_both made a plain call; redo the prepared one and compare its state
    assert reader.prepare_input(hidden, padding)
    out = reader(hidden, ids, weights, padding, input_prepared=True)
    torch.cuda.synchronize()
    assert_parity(reader, out, expected, tokens)


@pytest.mark.parametrize("tokens", [1, 20])
def test_prepared_input_runs_on_the_side_stream(tokens):
    """prepare_input rotates on the workspace's side stream while the current
    stream runs what the caller enqueues next (the router's place); the
    prepared call waits for it. Eagerly and captured in a HIP graph (the side
    stream forks from and joins the capture), replayed with new rows and
    padding, every result equals a plain call bit for bit."""
    layer = make_layer(hidden=512, width=256, experts=16, top_k=4, rank=16, tokens=tokens,
                       seed=110 + tokens)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    x = layer.hidden.to(DEVICE).clone()
    ids, weights = layer.ids.to(DEVICE), layer.weights.to(DEVICE)
    padding = torch.zeros(tokens, dtype=torch.bool, device=DEVICE)
    padding[-1] = tokens > 1
    router = torch.randn(512, 16, generator=torch.Generator().manual_seed(5)).to(DEVICE)
    assert reader.prepare_input(x, padding)
    side = reader.workspace.input_stream
    assert side is not None and side != torch.cuda.current_stream()
    logits = torch.mm(x.float(), router)
    prepared = reader(x, ids, weights, padding, input_prepared=True)
    torch.cuda.synchronize()
    assert not reader.workspace.input_pending
    plain = reader(x, ids, weights, padding)
    torch.cuda.synchronize()
    assert torch.equal(prepared, plain)
    assert torch.isfinite(logits).all()
    # a call that is not the prepared one still waits for a pending rotation
    # (of other rows here) before it rewrites the same workspace rows
    other = torch.randn(tokens, 512, generator=torch.Generator().manual_seed(9)).bfloat16().to(DEVICE)
    assert reader.prepare_input(other, padding)
    again = reader(x, ids, weights, padding)
    torch.cuda.synchronize()
    assert not reader.workspace.input_pending
    assert torch.equal(again, plain)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert reader.prepare_input(x, padding)
        scaled = x.float().mul(0.5)
        captured = reader(x, ids, weights, padding, input_prepared=True)
    generator = torch.Generator().manual_seed(11)
    for replay in range(3):
        x.copy_(torch.randn(tokens, 512, generator=generator).bfloat16())
        padding.zero_()
        padding[0] = replay == 1
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(scaled, x.float().mul(0.5))
        plain = reader(x, ids, weights, padding)
        torch.cuda.synchronize()
        assert torch.equal(captured, plain), f"replay {replay}"
    # the last plain call left this batch's state: the oracle holds it too
    _, expected = run_both(reader, layer, plan, x.cpu(), layer.ids, layer.weights, padding.cpu())
    assert reader.prepare_input(x, padding)
    out = reader(x, ids, weights, padding, input_prepared=True)
    torch.cuda.synchronize()
    assert_parity(reader, out, expected, tokens)


@pytest.mark.parametrize("tokens", [1, 3, 4])
@pytest.mark.parametrize("rank", [16, 32])
def test_select_and_exact_in_one_launch_equal_the_stages(tokens, rank):
    """Up to four tokens a full call runs select and exact as one launch: every
    workgroup selects, one stores the selection, the others compute the kept
    rows and (at rank 32) the recovery encoder items from their own copy of
    it. The stages relaunched one at a time run the separate kernels. Both
    leave the same outputs bit for bit, from stale flags too, and the call
    matches the oracle."""
    layer = make_layer(hidden=2048, width=768, experts=16, top_k=8, rank=rank, tokens=tokens,
                       seed=120 + tokens + rank)
    plan = compile_budget(hidden_size=2048, expert_width=768, top_k=8, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    hidden = layer.hidden.to(DEVICE)
    ids, weights = layer.ids.to(DEVICE), layer.weights.to(DEVICE)
    padding = torch.zeros(tokens, dtype=torch.bool, device=DEVICE)
    padding[-1] = tokens > 1
    names = ("selected", "completed", "partial", "counts", "starts", "tile_starts", "latent")

    def state():
        got = {name: getattr(reader, name)[:tokens].clone() for name in names}
        got["next_ids"] = reader.candidate_ids[-1][:tokens].clone()
        kept = got["completed"].bool()
        got["activations"] = torch.where(kept, reader.activations[:tokens], 0)
        return got

    out = reader(hidden, ids, weights, padding).clone()
    torch.cuda.synchronize()
    fused = state()
    # stale selection state: the stages rewrite all of it
    reader.selected.fill_(1)
    reader.completed.fill_(1)
    reader.candidate_ids[-1].fill_(-7)
    staged = torch.empty_like(out)
    for stage in _ext.STAGES:
        reader.launch_stage(stage, hidden, ids, weights, padding, staged)
    torch.cuda.synchronize()
    assert torch.equal(staged, out)
    for name, value in state().items():
        assert torch.equal(value, fused[name]), name
    # and the fused call again, from the same stale state
    reader.selected.fill_(1)
    reader.completed.fill_(1)
    reader.candidate_ids[-1].fill_(-7)
    _, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights, padding.cpu())
    out = reader(hidden, ids, weights, padding)
    torch.cuda.synchronize()
    assert_parity(reader, out, expected, tokens)


def test_prepare_input_is_a_no_op_for_a_dense_plan():
    layer = make_layer(hidden=256, width=64, experts=4, top_k=2, rank=8, tokens=2, seed=104)
    plan = compile_budget(hidden_size=256, expert_width=64, top_k=2, retention=1.0)
    reader = build(layer, plan, 2, selection_score="point")
    assert reader.prepare_input(layer.hidden.to(DEVICE)) is False


def test_default_constructor_builds_its_own_sketch():
    """sketch=None: the reader builds the codes from its device weights by the
    torch construction, so they are exactly `build_sketch` of the host weights
    (test_progressive_reader.py:803-805 of the reference), and screens with
    them; the oracle reads the same codes."""
    tokens = 3
    layer = make_layer(hidden=512, width=256, experts=8, top_k=4, rank=16, tokens=tokens,
                       seed=105)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = ProgressiveReader(
        layer.gate_up.to(DEVICE), channel_major_down(layer.down.to(DEVICE)),
        layer.encoder.to(DEVICE), layer.decoder.to(DEVICE), plan, tokens,
        selection_score="point",
    )
    # the reference's comparison of the two builds: codes exact, statistics
    # to atol 1e-4 / rtol 1e-3 (the device reduces in another order)
    assert torch.equal(reader.sketch_codes.cpu(), layer.codes)
    torch.testing.assert_close(reader.sketch_statistics.cpu(), layer.statistics, atol=1e-4, rtol=1e-3)
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


def test_qwen3_batch_128_bit_exact():
    """C3 at batch 128: 1,024 routed pairs over 128 experts (grouped paths)."""
    tokens = 128
    layer = make_layer(hidden=2048, width=768, experts=128, top_k=8, rank=32, tokens=tokens,
                       seed=73, device=DEVICE)
    plan = compile_budget(hidden_size=2048, expert_width=768, top_k=8, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, tokens, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, tokens)


@pytest.mark.parametrize("keep", [1.0, 0.625])
def test_fine_grained_experts_batch_1(keep):
    """C5 at batch 1: 256 experts of width 512 (block-paired sketch tails)."""
    layer = make_layer(hidden=2048, width=512, experts=256, top_k=8, rank=32, tokens=1,
                       seed=91, device=DEVICE)
    plan = compile_budget(hidden_size=2048, expert_width=512, top_k=8, retention=0.123,
                          screen_keep=keep)
    reader = build(layer, plan, 1, selection_score="point")
    out, expected = run_both(reader, layer, plan, layer.hidden, layer.ids, layer.weights)
    assert_parity(reader, out, expected, 1)
    assert int(reader.selected[0].sum()) == plan.final_count
    np.testing.assert_array_equal(expected["counts"].sum(1), plan.final_count)


def test_grouped_and_per_token_calls_agree_and_report_their_reads():
    """The same batch through per-token exact rows (grouped_tokens above the
    batch) and grouped ones (grouped_tokens = 2): identical results, identical
    read cost, and the requested bytes each kernel set reads (reference closed
    forms, tests/test_progressive_reader.py:959-978)."""
    tokens, experts, top_k, hidden, width, rank = 24, 16, 4, 512, 256, 16
    layer = make_layer(hidden=hidden, width=width, experts=experts, top_k=top_k, rank=rank,
                       tokens=tokens, seed=106)
    plan = compile_budget(hidden_size=hidden, expert_width=width, top_k=top_k,
                          retention=0.123, screen_keep=0.625)
    per_token = build(layer, plan, tokens, selection_score="point", grouped_tokens=tokens + 1)
    grouped = build(layer, plan, tokens, selection_score="point", grouped_tokens=2)
    hidden_rows = layer.hidden.to(DEVICE)
    ids, weights = layer.ids.to(DEVICE), layer.weights.to(DEVICE)
    padding = torch.tensor([t % 7 == 3 for t in range(tokens)], device=DEVICE)
    active = int((~padding).sum())
    a = per_token(hidden_rows, ids, weights, padding)
    b = grouped(hidden_rows, ids, weights, padding)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(per_token.selected[:tokens], grouped.selected[:tokens])
    token_report, grouped_report = per_token.report(), grouped.report()
    for key in ("charged_bytes", "logical_charged_bytes", "reference_bytes"):
        assert token_report[key] == grouped_report[key]
    assert grouped_report["grouped_rows"] == active and token_report["grouped_rows"] == 0
    # gate/up: every kept channel per token, or each tile's union once
    ws = grouped.workspace
    tiles = int(ws.group_total.item())
    masks = ws.tile_masks[: tiles * width].cpu().numpy().view(np.uint32)
    assert token_report["issued_gate_up_bytes"] == 4 * hidden * plan.final_count * active
    assert grouped_report["issued_gate_up_bytes"] == 4 * hidden * int((masks != 0).sum())
    assert grouped_report["issued_gate_up_bytes"] < token_report["issued_gate_up_bytes"]
    # down and encoder rows are requested per token in both
    for report in (token_report, grouped_report):
        assert report["issued_down_bytes"] == 2 * hidden * plan.final_count * active
        assert report["issued_recovery_encoder_bytes"] == 2 * rank * top_k * width * active
        # the screen streams each tile's trit planes and FP16 scales once
        blocks = hidden // 128
        assert report["issued_sketch_bytes"] == tiles * (64 * width * blocks + 4 * width * blocks)
        assert report["grouped_issued_matrix_macs"] == tiles * 2 * width * 16 * 128 * 3 * blocks
