"""Route traces: `.rrtrace` text format v1 (the normalised text form of a
`raggedroute.route_trace.v1` document, reference
configs/workloads/route_trace.schema.json).

Layout: the schema tag, the trace id, the source kind, one line
`T E top_k frames`, then one record per frame: its id followed by the frame's
T * top_k expert ids, token-major. Reading goes through the library's native
reader (`rr_route_trace_read`); `write` produces the same layout the
reference's normaliser writes, so a written trace reads back unchanged.
"""
from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass

import numpy as np

SCHEMA_TAG = "raggedroute.route_trace.v1"
SOURCE_KINDS = ("production", "captured", "synthetic_fixture")
MAX_EXPERTS = 1024  # the library's E cap (the schema's is 64)
_IDENT = re.compile(r"[A-Za-z0-9._-]+\Z")


@dataclass(frozen=True)
class RouteTrace:
    trace_id: str
    source_kind: str
    tokens: int
    experts: int
    top_k: int
    frame_count: int
    frame_id: str
    ids: np.ndarray  # [tokens, top_k] int32


def read(path, frame: int = 0) -> RouteTrace:
    """Frame `frame` of a trace file through the native reader; ValueError
    carries the reader's message when the file breaks the format."""
    import raggedroute_amd as rr

    info = rr.RouteTraceInfo()
    name = os.fsencode(path)
    status = rr.lib.rr_route_trace_read(name, frame, ctypes.byref(info), None, 0)
    if status.ok():
        ids = np.empty((info.tokens, info.top_k), np.int32)
        status = rr.lib.rr_route_trace_read(name, frame, ctypes.byref(info), ids.ctypes.data, ids.size)
    if not status.ok():
        raise ValueError(status.message)
    return RouteTrace(trace_id=info.trace_id.decode(), source_kind=info.source_kind.decode(),
                      tokens=info.tokens, experts=info.experts, top_k=info.top_k,
                      frame_count=info.frame_count, frame_id=info.frame_id.decode(), ids=ids)


def read_all(path) -> list[RouteTrace]:
    """Every frame of a trace file, in file order."""
    head = read(path, 0)
    return [head, *(read(path, f) for f in range(1, head.frame_count))]


def write(path, trace_id: str, source_kind: str, experts: int, frames: dict) -> str:
    """Write {frame_id: ids[T, top_k]} (one shape for every frame) as a v1
    text trace and return the text. Raises ValueError for input the reader
    would refuse, before anything is written."""
    if not _IDENT.match(trace_id):
        raise ValueError(f"trace id {trace_id!r}: letters, digits, '.', '_' and '-' only")
    if source_kind not in SOURCE_KINDS:
        raise ValueError(f"source kind {source_kind!r} is none of {', '.join(SOURCE_KINDS)}")
    if not frames:
        raise ValueError("a trace holds at least one frame")
    if not 1 <= experts <= MAX_EXPERTS:
        raise ValueError(f"E = {experts} outside [1, {MAX_EXPERTS}]")
    shape = None
    records = []
    for name, ids in frames.items():
        ids = np.asarray(ids)
        if not _IDENT.match(str(name)):
            raise ValueError(f"frame id {name!r}: letters, digits, '.', '_' and '-' only")
        if ids.ndim != 2 or ids.size == 0 or (shape is not None and ids.shape != shape):
            raise ValueError(f"frame {name}: ids must be one [T, top_k] shape for every frame")
        shape = ids.shape
        if not np.issubdtype(ids.dtype, np.integer) or ids.min() < 0 or ids.max() >= experts:
            raise ValueError(f"frame {name}: expert ids must be integers in [0, {experts})")
        ordered = np.sort(ids, axis=1)
        if (ordered[:, 1:] == ordered[:, :-1]).any():
            raise ValueError(f"frame {name}: a token names one expert twice")
        records.append(" ".join([str(name), *map(str, ids.reshape(-1).tolist())]))
    tokens, top_k = shape
    if top_k > experts:
        raise ValueError(f"top_k = {top_k} exceeds E = {experts}")
    text = "\n".join([SCHEMA_TAG, trace_id, source_kind,
                      f"{tokens} {experts} {top_k} {len(records)}", *records]) + "\n"
    with open(path, "w", encoding="ascii", newline="\n") as out:
        out.write(text)
    return text


def logits_for_ids(ids: np.ndarray, experts: int) -> np.ndarray:
    """chain_from_logits input under which the top-2 gate picks a frame's ids
    in order: -8 everywhere, +2 at each token's first id and +1 at its second
    (reference benchmarks/adapters/chain_adapter.cpp:209-230)."""
    ids = np.asarray(ids)
    if ids.ndim != 2 or ids.shape[1] != 2:
        raise ValueError("chain_from_logits replay needs a top_k = 2 trace")
    rows = np.arange(ids.shape[0])
    logits = np.full((ids.shape[0], experts), -8.0, np.float32)
    logits[rows, ids[:, 0]] = 2.0
    logits[rows, ids[:, 1]] = 1.0
    return logits
