"""Route traces: the `.rrtrace` text format v1 and its JSON form.

Reading a text trace goes through the library's native reader
(`rr_route_trace_read`, reference include/raggedroute/benchmark/adapter_utils.h:269-322).
The JSON form (reference configs/workloads/route_trace.schema.json) is validated
and normalised to text here, with the checks and error messages of reference
scripts/validate_route_trace.py:20-85; `python -m raggedroute_amd.route_trace
trace.json --output-normalized out.rrtrace` prints the same summary record.
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import pathlib
import re
import sys
from dataclasses import dataclass

import numpy as np

SCHEMA_VERSION = "raggedroute.route_trace.v1"
SOURCE_KINDS = ("production", "captured", "synthetic_fixture")
_PORTABLE = re.compile(r"[A-Za-z0-9._-]+")
MAX_EXPERTS = 1024  # the library's E cap (the reference's schema allows 64)


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
    """Frame `frame` of a text trace, through the native reader; raises
    ValueError with the reader's message on an invalid file."""
    import raggedroute_amd as rr

    info = rr.RouteTraceInfo()
    raw = str(path).encode()
    status = rr.lib.rr_route_trace_read(raw, frame, ctypes.byref(info), None, 0)
    if not status.ok():
        raise ValueError(status.message)
    ids = np.empty((info.tokens, info.top_k), np.int32)
    status = rr.lib.rr_route_trace_read(raw, frame, ctypes.byref(info), ids.ctypes.data, ids.size)
    if not status.ok():
        raise ValueError(status.message)
    return RouteTrace(info.trace_id.decode(), info.source_kind.decode(), info.tokens, info.experts,
                      info.top_k, info.frame_count, info.frame_id.decode(), ids)


def read_all(path) -> list[RouteTrace]:
    first = read(path, 0)
    return [first] + [read(path, f) for f in range(1, first.frame_count)]


def logits_for_ids(ids: np.ndarray, experts: int) -> np.ndarray:
    """chain_from_logits input that makes the top-2 gate pick a trace's ids in
    order: -8 everywhere, +2 at the first id and +1 at the second of each token
    (reference benchmarks/adapters/chain_adapter.cpp:209-230)."""
    ids = np.asarray(ids)
    if ids.ndim != 2 or ids.shape[1] != 2:
        raise ValueError("chain_from_logits replay needs a top_k = 2 trace")
    tokens = ids.shape[0]
    logits = np.full((tokens, experts), -8.0, np.float32)
    logits[np.arange(tokens), ids[:, 0]] = 2.0
    logits[np.arange(tokens), ids[:, 1]] = 1.0
    return logits


def _is_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def validate_trace(document) -> dict:
    """The JSON form's checks (reference scripts/validate_route_trace.py:20-71)."""
    if not isinstance(document, dict):
        raise ValueError("trace root must be an object")
    allowed = {"schema_version", "trace_id", "source_kind", "description", "anonymized",
               "tokens", "experts", "top_k", "frames"}
    unknown = sorted(set(document) - allowed)
    if unknown:
        raise ValueError(f"unknown trace fields: {', '.join(unknown)}")
    if document.get("schema_version") != SCHEMA_VERSION:
        raise ValueError(f"schema_version must be {SCHEMA_VERSION}")
    trace_id, kind = document.get("trace_id"), document.get("source_kind")
    tokens, experts, top_k = document.get("tokens"), document.get("experts"), document.get("top_k")
    frames = document.get("frames")
    if not isinstance(trace_id, str) or not _PORTABLE.fullmatch(trace_id):
        raise ValueError("trace_id must be a non-empty portable identifier")
    if kind not in SOURCE_KINDS:
        raise ValueError("source_kind must be production, captured, or synthetic_fixture")
    if not _is_int(tokens) or tokens < 1:
        raise ValueError("tokens must be a positive integer")
    if not _is_int(experts) or not 1 <= experts <= MAX_EXPERTS:
        raise ValueError(f"experts must be in [1, {MAX_EXPERTS}]")
    if not _is_int(top_k) or not 1 <= top_k <= experts:
        raise ValueError("top_k must satisfy 1<=top_k<=experts")
    if not isinstance(frames, list) or not frames:
        raise ValueError("frames must be a non-empty array")
    routes = tokens * top_k
    seen = set()
    for index, frame in enumerate(frames):
        if not isinstance(frame, dict) or set(frame) != {"frame_id", "expert_ids"}:
            raise ValueError(f"frame {index} must contain only frame_id and expert_ids")
        fid, ids = frame["frame_id"], frame["expert_ids"]
        if not isinstance(fid, str) or not _PORTABLE.fullmatch(fid):
            raise ValueError(f"frame {index} has an invalid frame_id")
        if fid in seen:
            raise ValueError(f"duplicate frame_id: {fid}")
        seen.add(fid)
        if not isinstance(ids, list) or len(ids) != routes:
            raise ValueError(f"frame {fid} must contain {routes} expert ids")
        if not all(_is_int(v) and 0 <= v < experts for v in ids):
            raise ValueError(f"frame {fid} contains an out-of-range expert id")
        for t in range(tokens):
            if len(set(ids[t * top_k:(t + 1) * top_k])) != top_k:
                raise ValueError(f"frame {fid} token {t} repeats an expert")
    return document


def normalized_text(document: dict) -> str:
    """Text form: schema, id, kind, `T E top_k frames`, one line per frame."""
    lines = [SCHEMA_VERSION, document["trace_id"], document["source_kind"],
             f'{document["tokens"]} {document["experts"]} {document["top_k"]} {len(document["frames"])}']
    lines += [f["frame_id"] + " " + " ".join(str(v) for v in f["expert_ids"]) for f in document["frames"]]
    return "\n".join(lines) + "\n"


def document(trace_id: str, source_kind: str, experts: int, frames: dict) -> dict:
    """JSON document from {frame_id: ids[tokens, top_k]} (all frames one shape)."""
    arrays = [np.asarray(v) for v in frames.values()]
    tokens, top_k = arrays[0].shape
    return validate_trace({
        "schema_version": SCHEMA_VERSION, "trace_id": trace_id, "source_kind": source_kind,
        "tokens": int(tokens), "experts": int(experts), "top_k": int(top_k),
        "frames": [{"frame_id": k, "expert_ids": [int(x) for x in np.asarray(v).reshape(-1)]}
                   for k, v in frames.items()]})


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Validate and normalise a JSON route trace.")
    ap.add_argument("trace", type=pathlib.Path)
    ap.add_argument("--output-normalized", type=pathlib.Path)
    ap.add_argument("--require-real", action="store_true", help="reject source_kind=synthetic_fixture")
    args = ap.parse_args(argv)
    doc = validate_trace(json.loads(args.trace.read_text(encoding="utf-8")))
    if args.require_real and doc["source_kind"] == "synthetic_fixture":
        raise ValueError("real-trace evaluation rejects synthetic_fixture input")
    text = normalized_text(doc)
    if args.output_normalized:
        args.output_normalized.parent.mkdir(parents=True, exist_ok=True)
        args.output_normalized.write_text(text, encoding="utf-8", newline="\n")
    print(json.dumps({"schema_version": SCHEMA_VERSION, "trace_id": doc["trace_id"],
                      "source_kind": doc["source_kind"], "tokens": doc["tokens"],
                      "experts": doc["experts"], "top_k": doc["top_k"], "frames": len(doc["frames"]),
                      "normalized_sha256": hashlib.sha256(text.encode("utf-8")).hexdigest()},
                     sort_keys=True))
    return 0


if __name__ == "__main__":
    try:
        raise SystemExit(main())
    except Exception as error:  # noqa: BLE001  (CLI: message + exit code 2)
        print(f"error: {error}", file=sys.stderr)
        raise SystemExit(2)
