"""ctypes front end of the CPU oracle (oracle/cfmoe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, `__graft_entry__.smoke()` and the
CPU-baseline leg of bench.py as the checker. The reader's product path never
imports this module.

Every function takes and returns numpy arrays. BF16 tensors travel as their
uint16 bit patterns, FP16 statistics likewise. `forward` runs the whole reader
for one call and returns every intermediate the HIP reader also exposes.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib: ctypes.CDLL | None = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile; return its path."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_expf.restype = ctypes.c_float
        _lib.orc_expf.argtypes = [ctypes.c_float]
        _lib.orc_sigmoid.restype = ctypes.c_float
        _lib.orc_sigmoid.argtypes = [ctypes.c_float]
        _lib.orc_activate.restype = ctypes.c_float
        _lib.orc_activate.argtypes = [ctypes.c_float, ctypes.c_int]
        _lib.orc_score_one.restype = ctypes.c_float
        _lib.orc_score_one.argtypes = [ctypes.c_float] * 8 + [ctypes.c_int] * 2
        _lib.orc_code_stride.restype = ctypes.c_int
        _lib.orc_storage_bytes.restype = ctypes.c_long
        _lib.orc_row_dot.restype = ctypes.c_float
    return _lib


def _p(array: np.ndarray | None):
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return array.ctypes.data_as(ctypes.c_void_p)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round FP32 values to BF16 (nearest even) and return the uint16 bits."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    rounded = np.where(nan, (bits >> 16) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(
        np.float32
    )


def expf(x: float) -> float:
    return lib().orc_expf(x)


def activate(g: float, gelu: bool = False) -> float:
    return lib().orc_activate(g, int(gelu))


def score_one(gate, up, gate_variance, up_variance, norm, weight, alpha, beta,
              gelu=False, point=True) -> float:
    return lib().orc_score_one(gate, up, gate_variance, up_variance, norm, weight,
                               alpha, beta, int(gelu), int(point))


def row_dot(row_bits: np.ndarray, x_bits: np.ndarray) -> float:
    row_bits = np.ascontiguousarray(row_bits, dtype=np.uint16)
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    return lib().orc_row_dot(ctypes.c_int(len(row_bits)), _p(row_bits), _p(x_bits))


def route(router_ids: np.ndarray, router_weights: np.ndarray, padding=None, experts=1 << 30):
    t, k = router_ids.shape
    ids = np.empty((t, k), np.int32)
    weights = np.empty((t, k), np.float32)
    rid = np.ascontiguousarray(router_ids, dtype=np.int64)
    rw = np.ascontiguousarray(router_weights, dtype=np.float32)
    pad = None if padding is None else np.ascontiguousarray(padding, dtype=np.uint8)
    lib().orc_route(t, k, experts, _p(rid), _p(rw), _p(pad), _p(ids), _p(weights))
    return ids, weights


def rotate(x_bits: np.ndarray, signs: np.ndarray, keep: int, padding=None):
    t, h = x_bits.shape
    b = h // 128
    planes = np.empty((t, b, keep), np.float32)
    coords = np.empty((t, b, keep), np.int32)
    qvals = np.empty((t, b, keep), np.int32)
    qexp = np.empty((t, b), np.int32)
    norm2 = np.empty((t, b), np.float32)
    xb = np.ascontiguousarray(x_bits, dtype=np.uint16)
    sg = np.ascontiguousarray(signs, dtype=np.int8)
    pad = None if padding is None else np.ascontiguousarray(padding, dtype=np.uint8)
    lib().orc_rotate(t, h, keep, _p(xb), _p(sg), _p(pad), _p(planes), _p(coords),
                     _p(qvals), _p(qexp), _p(norm2))
    return planes, coords, qvals, qexp, norm2


@dataclass
class Weights:
    """One layer's reader inputs as numpy arrays (BF16/FP16 as bit patterns)."""

    gate_up: np.ndarray  # [E, 2I, H] uint16
    down: np.ndarray  # physical [E, I, H] uint16 (channel-major)
    codes: np.ndarray  # [E, storage] uint8
    stats: np.ndarray  # physical [E, B, 2, 2I] uint16 (fp16 bits)
    norms: np.ndarray  # [E, I] float32
    signs: np.ndarray  # [H] int8
    encoder_t: np.ndarray | None = None  # [E, I, R] uint16
    decoder: np.ndarray | None = None  # [H, R] uint16
    geometry: np.ndarray | None = None  # [E, I, 2] float32


def forward(w: Weights, x_bits, router_ids, router_weights, *, final_count: int,
            keep: int, padding=None, point: bool = True, gelu: bool = False,
            threshold: float | None = None, threads: int = 1) -> dict[str, np.ndarray]:
    """Run the whole reader for one call; returns every intermediate.

    `threads` OpenMP threads split the screen's rows, the kept channels and
    the down outputs (the results do not depend on it).
    """
    L = lib()
    T, H = x_bits.shape
    E, rows, _ = w.gate_up.shape
    I = rows // 2
    K = router_ids.shape[1]
    N, F = K * I, final_count
    R = 0 if w.decoder is None else w.decoder.shape[1]
    pad = None if padding is None else np.ascontiguousarray(padding, dtype=np.uint8)
    ids, weights = route(router_ids, router_weights, pad, E)
    planes, coords, qvals, qexp, norm2 = rotate(x_bits, w.signs, keep, pad)
    partial = np.zeros((T, 2, N), np.float32)
    variances = np.zeros((T, 2, N), np.float32)
    screened = F < N
    if screened:
        L.orc_screen(T, H, I, K, keep, _p(w.codes), _p(w.stats), _p(coords), _p(qvals),
                     _p(qexp), _p(norm2), _p(ids), _p(pad), _p(partial), _p(variances),
                     int(threads))
    scores = np.zeros((T, N), np.float32)
    next_ids = np.empty((T, F), np.int32)
    selected = np.zeros((T, N), np.uint8)
    counts = np.empty((T, K), np.int32)
    starts = np.empty((T, K), np.int32)
    tile_starts = np.empty((T, K), np.int32)
    if screened:
        L.orc_score(T, I, K, _p(partial), _p(variances), _p(ids), _p(weights), _p(pad),
                    _p(w.norms), _p(w.geometry), int(gelu), int(point), _p(scores))
        L.orc_select(T, N, F, I, K, _p(scores), int(threshold is not None),
                     ctypes.c_float(0.0 if threshold is None else threshold),
                     _p(next_ids), _p(selected), _p(counts), _p(starts), _p(tile_starts))
    else:
        next_ids[:] = np.arange(N, dtype=np.int32)
        selected[:] = 1
        counts[:] = I
        starts[:] = np.arange(K, dtype=np.int32) * I
        tile_starts[:] = np.arange(K, dtype=np.int32) * ((I + 127) // 128)
    activations = np.zeros((T, N), np.uint16)
    completed = np.zeros((T, N), np.uint8)
    xb = np.ascontiguousarray(x_bits, dtype=np.uint16)
    L.orc_exact(T, H, I, K, F, _p(w.gate_up), _p(xb), _p(ids), _p(pad), _p(next_ids),
                int(gelu), _p(partial), _p(activations), _p(completed), int(threads))
    values = np.empty((T, K, H), np.float32)
    L.orc_down(T, H, I, K, F, _p(w.down), _p(activations), _p(ids), _p(pad),
               _p(next_ids), _p(counts), _p(starts), _p(values), int(threads))
    latent = np.zeros((T, max(R, 1)), np.float32)
    if R:
        L.orc_encode(T, I, K, R, _p(w.encoder_t), _p(partial), _p(activations),
                     _p(completed), _p(selected), _p(ids), _p(weights), _p(pad),
                     int(gelu), _p(latent))
    out = np.empty((T, H), np.uint16)
    L.orc_output(T, H, K, R, _p(values), _p(weights), _p(latent), _p(w.decoder),
                 _p(pad), _p(out))
    return {
        "ids": ids, "weights": weights, "planes": planes, "coordinates": coords,
        "qvals": qvals, "qexp": qexp, "norm2": norm2, "partial": partial,
        "variances": variances, "scores": scores, "next_ids": next_ids,
        "selected": selected, "counts": counts, "starts": starts,
        "tile_starts": tile_starts, "activations": activations,
        "completed": completed, "values": values, "latent": latent[:, :R],
        "out": out,
    }


def forward_parallel(w: Weights, x_bits, router_ids, router_weights, *, padding=None,
                     workers: int | None = None, **options) -> dict[str, np.ndarray]:
    """`forward` over contiguous token ranges in threads, results concatenated.

    Every stage of the reader is per token (a token's routing, screen,
    selection, exact rows, down sums, latent and output read no other token's
    values), so the ranges' results are the whole call's. ctypes releases the
    GIL during each C call, so the ranges run on separate cores.
    """
    from concurrent.futures import ThreadPoolExecutor

    tokens = x_bits.shape[0]
    workers = max(1, min(workers or os.cpu_count() or 1, 16, tokens))
    bounds = np.linspace(0, tokens, workers + 1).astype(int)
    ranges = [(lo, hi) for lo, hi in zip(bounds[:-1], bounds[1:]) if hi > lo]

    def run(span):
        lo, hi = span
        return forward(w, np.ascontiguousarray(x_bits[lo:hi]),
                       np.ascontiguousarray(router_ids[lo:hi]),
                       np.ascontiguousarray(router_weights[lo:hi]),
                       padding=None if padding is None else np.ascontiguousarray(padding[lo:hi]),
                       **options)

    with ThreadPoolExecutor(len(ranges)) as pool:
        parts = list(pool.map(run, ranges))
    return {key: np.concatenate([part[key] for part in parts]) for key in parts[0]}
