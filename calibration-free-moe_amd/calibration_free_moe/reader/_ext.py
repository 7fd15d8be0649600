"""ctypes binding of libcfmoe_reader.so (C ABI declared in include/cfmoe_reader.h).

The shared library is built in-tree next to this file (see `__graft_entry__.
build()` at the repository root). There is no fallback: if it is missing or
fails to load, every reader call raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os

LIBRARY_NAME = "libcfmoe_reader.so"
LIBRARY_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)

ABI_VERSION = 10

POINT = 1
GELU = 2
GEOMETRY = 4
THRESHOLD = 8
ACCOUNT = 16
IDS_INT64 = 32
WEIGHTS_BF16 = 64
INPUT_PREPARED = 128

EINVAL = 1
EHIP = 2

STAGES = ("prepare", "screen", "score", "select", "exact", "encode", "down", "output")

# Batch size from which the screen stage launches fused_screen_kernel (below
# it, small_screen_kernel); kFusedScreenTokens in csrc/cfmoe_reader.hip.
FUSED_SCREEN_TOKENS = 2


class Dims(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("experts", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("final_count", ctypes.c_int32),
        ("keep", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("grouped_tokens", ctypes.c_int32),
    ]


class WeightPointers(ctypes.Structure):
    _fields_ = [
        ("gate_up", ctypes.c_void_p),
        ("down", ctypes.c_void_p),
        ("codes", ctypes.c_void_p),
        ("statistics", ctypes.c_void_p),
        ("norms", ctypes.c_void_p),
        ("geometry", ctypes.c_void_p),
        ("encoder_t", ctypes.c_void_p),
        ("decoder", ctypes.c_void_p),
        ("signs", ctypes.c_void_p),
        ("threshold", ctypes.c_void_p),
        ("trit_planes", ctypes.c_void_p),
        ("encoder_tiles", ctypes.c_void_p),
    ]


# Workspace buffers in C struct order (after `capacity`), with element dtypes.
WORKSPACE_FIELDS = (
    ("ids", "int32"),
    ("weights", "float32"),
    ("planes", "float32"),
    ("coordinates", "int32"),
    ("qvals", "int32"),
    ("qexp", "int32"),
    ("qsums", "int32"),
    ("norm2", "float32"),
    ("partial", "float32"),
    ("variances", "float32"),
    ("scores", "float32"),
    ("next_ids", "int32"),
    ("selected", "bool"),
    ("completed", "bool"),
    ("activations", "bfloat16"),
    ("starts", "int32"),
    ("counts", "int32"),
    ("tile_starts", "int32"),
    ("down_tile_starts", "int32"),
    ("down_parts", "float32"),
    ("encoder_parts", "float32"),
    ("latent", "float32"),
    ("group_experts", "int32"),
    ("group_starts", "int32"),
    ("group_counts", "int32"),
    ("group_pairs", "int32"),
    ("group_total", "int32"),
    ("pair_tiles", "int32"),
    ("tile_masks", "int32"),
    ("down_order", "int32"),
    ("digits", "int8"),
)


class WorkspacePointers(ctypes.Structure):
    _fields_ = [("capacity", ctypes.c_int32)] + [
        (name, ctypes.c_void_p) for name, _ in WORKSPACE_FIELDS
    ] + [("read_work", ctypes.c_void_p)]


_library: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load the HIP reader library once; raise RuntimeError if it is absent."""
    global _library
    if _library is not None:
        return _library
    if not os.path.exists(LIBRARY_PATH):
        raise RuntimeError(
            f"{LIBRARY_NAME} is not built; run `python -c 'import __graft_entry__ as g; "
            "g.build()'` at the repository root (hipcc --offload-arch=gfx950)"
        )
    lib = ctypes.CDLL(LIBRARY_PATH)
    lib.cfmoe_abi_version.restype = ctypes.c_int
    lib.cfmoe_last_error.restype = ctypes.c_char_p
    lib.cfmoe_workspace_sizes.restype = ctypes.c_int
    lib.cfmoe_workspace_sizes.argtypes = [
        ctypes.POINTER(Dims), ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32
    ]
    lib.cfmoe_forward.restype = ctypes.c_int
    lib.cfmoe_forward.argtypes = [
        ctypes.POINTER(Dims),
        ctypes.POINTER(WeightPointers),
        ctypes.POINTER(WorkspacePointers),
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_int32,
        ctypes.POINTER(ctypes.c_double),
        ctypes.c_void_p,
    ]
    lib.cfmoe_launch_stage.restype = ctypes.c_int
    lib.cfmoe_launch_stage.argtypes = [ctypes.c_int32] + lib.cfmoe_forward.argtypes
    lib.cfmoe_trit_plane_bytes.restype = ctypes.c_int64
    lib.cfmoe_trit_plane_bytes.argtypes = [ctypes.POINTER(Dims)]
    lib.cfmoe_pack_trit_planes.restype = ctypes.c_int
    lib.cfmoe_pack_trit_planes.argtypes = [
        ctypes.POINTER(Dims), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p
    ]
    lib.cfmoe_unpack_trit_planes.restype = ctypes.c_int
    lib.cfmoe_unpack_trit_planes.argtypes = [
        ctypes.POINTER(Dims), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p
    ]
    lib.cfmoe_build_sketch.restype = ctypes.c_int
    lib.cfmoe_build_sketch.argtypes = [
        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
    ]
    lib.cfmoe_prepare_input.restype = ctypes.c_int
    lib.cfmoe_prepare_input.argtypes = [
        ctypes.POINTER(Dims),
        ctypes.POINTER(WeightPointers),
        ctypes.POINTER(WorkspacePointers),
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_int32,
        ctypes.c_void_p,
    ]
    if lib.cfmoe_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIBRARY_NAME} ABI mismatch; rebuild the library")
    _library = lib
    return lib


def check(status: int) -> None:
    """Turn a nonzero C status into ValueError (contract) or RuntimeError (HIP)."""
    if status == 0:
        return
    message = library().cfmoe_last_error().decode(errors="replace")
    if status == EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def workspace_sizes(dims: Dims, capacity: int) -> list[int]:
    sizes = (ctypes.c_int64 * len(WORKSPACE_FIELDS))()
    written = library().cfmoe_workspace_sizes(
        ctypes.byref(dims), capacity, sizes, len(WORKSPACE_FIELDS)
    )
    if written < 0:
        check(-written)
    return list(sizes)


def trit_plane_bytes(dims: Dims) -> int:
    size = library().cfmoe_trit_plane_bytes(ctypes.byref(dims))
    if size < 0:
        check(-size)
    return size
