"""cfmoe_forward_noalloc against cfmoe_forward (needs an MI355X).

The allocation-free entry point carves its workspace from a static device
array; its results must equal the workspace entry point's bit for bit, on two
calls in a row, the second with fewer tokens (the array keeps the first call's
contents), including the read statistics. Oversized calls are rejected before
any device work.
"""

import ctypes

import pytest
import torch

from calibration_free_moe.reader import _ext
from calibration_free_moe.reader.budget import compile_budget
from tests.synthetic import make_layer
from tests.test_gpu_parity import DEVICE, build

pytestmark = pytest.mark.gpu


def noalloc(reader, hidden, ids, weights, padding, out, read_work):
    lib = _ext.library()
    lib.cfmoe_forward_noalloc.restype = ctypes.c_int
    tokens = hidden.shape[0]
    dims = reader._call_dims(ids, weights, False)
    status = lib.cfmoe_forward_noalloc(
        ctypes.byref(dims), ctypes.byref(reader._weights_c), ctypes.c_void_p(hidden.data_ptr()),
        ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(weights.data_ptr()),
        None if padding is None else ctypes.c_void_p(padding.data_ptr()),
        ctypes.c_void_p(out.data_ptr()), ctypes.c_int32(tokens),
        ctypes.c_void_p(read_work.data_ptr()), reader._charges[tokens >= reader.grouped_tokens],
        ctypes.c_void_p(torch.cuda.current_stream(DEVICE).cuda_stream))
    return status


@pytest.mark.parametrize("score", ["point", "recovery-aware"])
def test_noalloc_matches_the_workspace_entry_point(score):
    first_tokens, second_tokens = 24, 3
    layer = make_layer(hidden=512, width=256, experts=16, top_k=4, rank=32,
                       tokens=first_tokens, seed=120)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, first_tokens, selection_score=score)
    hidden = layer.hidden.to(DEVICE)
    ids, weights = layer.ids.to(DEVICE), layer.weights.to(DEVICE)
    padding = torch.zeros(first_tokens, dtype=torch.bool, device=DEVICE)
    padding[5] = True
    for tokens in (first_tokens, second_tokens):
        rows = slice(0, tokens)
        reader.read_work.zero_()
        want = reader(hidden[rows], ids[rows], weights[rows], padding[rows])
        read_work = torch.zeros(20, dtype=torch.float64, device=DEVICE)
        got = torch.full_like(want, float("nan"))
        status = noalloc(reader, hidden[rows], ids[rows].contiguous(),
                         weights[rows].contiguous(), padding[rows], got, read_work)
        torch.cuda.synchronize()
        assert status == 0, _ext.library().cfmoe_last_error()
        assert torch.equal(got, want), tokens
        assert torch.equal(read_work, reader.read_work), tokens


def test_noalloc_rejects_calls_beyond_its_array():
    layer = make_layer(hidden=512, width=256, experts=16, top_k=4, rank=32, tokens=2, seed=121)
    plan = compile_budget(hidden_size=512, expert_width=256, top_k=4, retention=0.123,
                          screen_keep=0.625)
    reader = build(layer, plan, 2, selection_score="point")
    lib = _ext.library()
    lib.cfmoe_noalloc_scratch_bytes.restype = ctypes.c_int64
    assert lib.cfmoe_noalloc_scratch_bytes() == 64 << 20
    dims = reader._call_dims(layer.ids, layer.weights, False)
    dims.flags &= ~_ext.ACCOUNT
    lib.cfmoe_forward_noalloc.restype = ctypes.c_int
    fake = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    status = lib.cfmoe_forward_noalloc(ctypes.byref(dims), ctypes.byref(reader._weights_c), fake,
                                       fake, fake, None, fake, ctypes.c_int32(2048), None, None,
                                       None)
    assert status == _ext.EINVAL
    assert b"allocation-free entry point holds" in lib.cfmoe_last_error()
