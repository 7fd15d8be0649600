"""The C-ABI library loads and exports every entry point include/cfmoe_reader.h
declares (no compute call: this runs without a GPU)."""

import ctypes
import os
import re

import pytest

from calibration_free_moe.reader import _ext
from calibration_free_moe.reader.budget import compile_budget

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "cfmoe_reader.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:CFMOE_API\s+)?(?:const\s+)?\w+\s*\*?\s*(cfmoe_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _ext.library()
    names = declared_functions()
    assert {"cfmoe_forward", "cfmoe_prepare_input", "cfmoe_launch_stage",
            "cfmoe_workspace_sizes", "cfmoe_last_error", "cfmoe_abi_version"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.cfmoe_abi_version() == _ext.ABI_VERSION


def test_workspace_sizes_and_contract_errors():
    plan = compile_budget(hidden_size=2048, expert_width=768, top_k=8, retention=0.123,
                          screen_keep=0.625)
    dims = _ext.Dims(2048, 768, 8, 128, 32, plan.final_count, 80, 0)
    sizes = _ext.workspace_sizes(dims, 4)
    names = [name for name, _ in _ext.WORKSPACE_FIELDS]
    assert sizes[names.index("partial")] == 4 * 2 * 6144 * 4
    assert sizes[names.index("next_ids")] == 4 * plan.final_count * 4
    bad = _ext.Dims(2000, 768, 8, 128, 32, 10, 80, 0)
    with pytest.raises(ValueError, match="multiple of 128"):
        _ext.workspace_sizes(bad, 4)
    # hidden sizes up to 4096 (Gemma 4's 2816 among them) are accepted, wider ones refused
    for hidden in (2816, 4096):
        _ext.workspace_sizes(_ext.Dims(hidden, 704, 2, 4, 32, 100, 80, 0), 4)
    with pytest.raises(ValueError, match="at most 4096"):
        _ext.workspace_sizes(_ext.Dims(4224, 704, 2, 4, 32, 100, 80, 0), 4)
    _ext.workspace_sizes(_ext.Dims(2048, 2048, 8, 4, 32, 100, 80, 0), 4)
    with pytest.raises(ValueError, match="at most 2048"):
        _ext.workspace_sizes(_ext.Dims(2048, 2064, 2, 4, 32, 100, 80, 0), 4)


def test_forward_rejects_null_arguments_without_touching_a_device():
    lib = _ext.library()
    dims = _ext.Dims(256, 64, 2, 4, 0, 16, 80, 0)
    weights = _ext.WeightPointers()
    workspace = _ext.WorkspacePointers()
    workspace.capacity = 1
    status = lib.cfmoe_forward(ctypes.byref(dims), ctypes.byref(weights),
                               ctypes.byref(workspace), None, None, None, None, None, 1,
                               None, None)
    assert status == _ext.EINVAL
    assert b"NULL" in lib.cfmoe_last_error()


def test_forward_rejects_misaligned_projections_without_touching_a_device():
    lib = _ext.library()
    dims = _ext.Dims(256, 64, 2, 4, 0, 16, 80, 0)
    weights = _ext.WeightPointers()
    weights.trit_planes = 0x4000
    weights.statistics = 0x5000
    weights.norms = 0x6000
    workspace = _ext.WorkspacePointers()
    workspace.capacity = 1
    workspace.partial = 0x1000 + 4
    workspace.variances = 0x2000
    workspace.scores = 0x3000
    workspace.digits = 0x7000
    fake = ctypes.c_void_p(0x8000)
    status = lib.cfmoe_forward(ctypes.byref(dims), ctypes.byref(weights),
                               ctypes.byref(workspace), fake, fake, fake, None, fake, 1,
                               None, None)
    assert status == _ext.EINVAL
    assert b"16-byte aligned" in lib.cfmoe_last_error()


def test_forward_refuses_a_grouped_size_of_one_token():
    """A 1-token call runs the per-token screen, which leaves the tile masks of
    the grouped exact rows as they are; grouped_tokens = 1 is refused before
    any device work (0 keeps the default, 2 and more are accepted)."""
    lib = _ext.library()
    weights = _ext.WeightPointers()
    workspace = _ext.WorkspacePointers()
    workspace.capacity = 1
    for grouped, refused in ((1, True), (-3, True), (0, False), (2, False)):
        dims = _ext.Dims(256, 64, 2, 4, 0, 16, 80, 0, grouped)
        status = lib.cfmoe_forward(ctypes.byref(dims), ctypes.byref(weights),
                                   ctypes.byref(workspace), None, None, None, None, None, 1,
                                   None, None)
        assert status == _ext.EINVAL
        message = lib.cfmoe_last_error()
        assert (b"grouped_tokens" in message) == refused, message
        if not refused:
            assert b"NULL" in message
