"""Route traces on the host: the native `.rrtrace` reader (rr_route_trace_read)
against the reference's fixture and planted format errors (reference
include/raggedroute/benchmark/adapter_utils.h:269-322), and the JSON form's
validator / normaliser (reference scripts/validate_route_trace.py). CPU only.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
import raggedroute_amd as rr
from raggedroute_amd import route_trace

FIXTURE = Path(__file__).resolve().parent / "golden" / "synthetic_fixture.rrtrace"
FRAMES = ("balanced", "skewed", "shifted")


def test_fixture_frames_match_the_golden_vectors(kat):
    raw = kat.raw["route_trace_fixture"]
    for index, name in enumerate(FRAMES):
        tr = route_trace.read(FIXTURE, index)
        assert (tr.trace_id, tr.source_kind, tr.frame_id) == (raw["trace_id"], raw["source_kind"], name)
        assert (tr.tokens, tr.experts, tr.top_k, tr.frame_count) == (8, 8, 2, 3)
        assert tr.ids.dtype == np.int32 and tr.ids.shape == (8, 2)
        assert tr.ids.reshape(-1).tolist() == raw["frames"][name]
    assert [t.frame_id for t in route_trace.read_all(FIXTURE)] == list(FRAMES)


def test_header_only_read_and_small_buffer():
    info = rr.RouteTraceInfo()
    st = rr.lib.rr_route_trace_read(str(FIXTURE).encode(), 2, ctypes.byref(info), None, 0)
    assert st.ok() and info.frame_id == b"shifted" and info.frame_count == 3
    buf = np.full(15, -7, np.int32)
    st = rr.lib.rr_route_trace_read(str(FIXTURE).encode(), 0, ctypes.byref(info), buf.ctypes.data, 15)
    assert st.code == rr.StatusCode.kInvalidArgument and (buf == -7).all()


def _write(tmp_path, text, name="t.rrtrace"):
    p = tmp_path / name
    p.write_text(text)
    return p


GOOD = FIXTURE.read_text()


@pytest.mark.parametrize("mutate,message", [
    (lambda s: s.replace("raggedroute.route_trace.v1", "raggedroute.route_trace.v2"), "header"),
    (lambda s: s.replace("synthetic_fixture_t8_e8_top2", "bad id!"), "metadata"),
    (lambda s: s.replace("\nsynthetic_fixture\n", "\nsynthetic\n"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "0 8 2 3"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "8 0 2 3"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "8 1025 2 3"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "8 8 9 3"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "8 8 2 0"), "metadata"),
    (lambda s: s.replace("8 8 2 3", "8 8 2"), "header"),
    (lambda s: s.replace("skewed", "balanced"), "frame id"),
    (lambda s: s.replace("skewed", "sk/ewed"), "frame id"),
    (lambda s: s.replace("balanced 0 1", "balanced 0 8"), "expert id"),
    (lambda s: s.replace("balanced 0 1", "balanced -1 1"), "expert id"),
    (lambda s: s.replace("balanced 0 1", "balanced 0 x"), "expert id"),
    (lambda s: s.replace("balanced 0 1", "balanced 1 1"), "repeats an expert"),
    (lambda s: s.replace("shifted 7 6", "shifted 7 7"), "repeats an expert"),
    (lambda s: s + "extra\n", "trailing"),
    (lambda s: s.rsplit(" ", 1)[0] + "\n", "expert id"),
])
def test_reader_rejects_planted_errors(tmp_path, mutate, message):
    bad = mutate(GOOD)
    assert bad != GOOD
    with pytest.raises(ValueError, match=message):
        route_trace.read(_write(tmp_path, bad), 0)


def test_reader_argument_errors(tmp_path):
    with pytest.raises(ValueError, match="cannot open"):
        route_trace.read(tmp_path / "missing.rrtrace", 0)
    with pytest.raises(ValueError, match="metadata"):
        route_trace.read(FIXTURE, 3)  # frame past the last
    with pytest.raises(ValueError, match="invalid"):
        route_trace.read(FIXTURE, -1)


def test_error_in_a_later_frame_leaves_the_buffer_untouched(tmp_path):
    bad = _write(tmp_path, GOOD.replace("shifted 7 6", "shifted 7 7"))
    info = rr.RouteTraceInfo()
    buf = np.full(16, -5, np.int32)
    st = rr.lib.rr_route_trace_read(str(bad).encode(), 0, ctypes.byref(info), buf.ctypes.data, 16)
    assert st.code == rr.StatusCode.kInvalidArgument and (buf == -5).all()


def test_json_round_trip_and_cli(tmp_path, kat, capsys):
    raw = kat.raw["route_trace_fixture"]
    doc = route_trace.document(raw["trace_id"], raw["source_kind"], raw["experts"],
                               {f: np.array(raw["frames"][f]).reshape(8, 2) for f in FRAMES})
    assert route_trace.normalized_text(doc) == GOOD  # byte-identical to the reference fixture
    src = tmp_path / "trace.json"
    src.write_text(json.dumps(doc))
    out = tmp_path / "norm" / "trace.rrtrace"
    assert route_trace.main([str(src), "--output-normalized", str(out)]) == 0
    summary = json.loads(capsys.readouterr().out)
    assert summary["normalized_sha256"] == hashlib.sha256(GOOD.encode()).hexdigest()
    assert summary["frames"] == 3 and out.read_text() == GOOD
    assert route_trace.read(out, 1).ids.reshape(-1).tolist() == raw["frames"]["skewed"]
    with pytest.raises(ValueError, match="synthetic_fixture"):
        route_trace.main([str(src), "--require-real"])


@pytest.mark.parametrize("edit,message", [
    (lambda d: d.update(extra=1), "unknown trace fields"),
    (lambda d: d.update(schema_version="v0"), "schema_version"),
    (lambda d: d.update(trace_id="a b"), "trace_id"),
    (lambda d: d.update(source_kind="lab"), "source_kind"),
    (lambda d: d.update(tokens=True), "tokens"),
    (lambda d: d.update(experts=2000), "experts"),
    (lambda d: d.update(top_k=9), "top_k"),
    (lambda d: d.update(frames=[]), "frames"),
    (lambda d: d["frames"][0].update(weight=1), "only frame_id and expert_ids"),
    (lambda d: d["frames"][1].update(frame_id="balanced"), "duplicate frame_id"),
    (lambda d: d["frames"][0].update(expert_ids=[0] * 15), "must contain 16"),
    (lambda d: d["frames"][0]["expert_ids"].__setitem__(3, 8), "out-of-range"),
    (lambda d: d["frames"][0]["expert_ids"].__setitem__(1, 0), "repeats an expert"),
])
def test_json_validator_rejects(kat, edit, message):
    raw = kat.raw["route_trace_fixture"]
    doc = json.loads(json.dumps(route_trace.document(
        raw["trace_id"], raw["source_kind"], raw["experts"],
        {f: np.array(raw["frames"][f]).reshape(8, 2) for f in FRAMES})))
    edit(doc)
    with pytest.raises(ValueError, match=message):
        route_trace.validate_trace(doc)


def test_logits_for_ids_select_the_trace_ids(kat):
    """The replay logits make the oracle top-2 return the frame's ids in order
    with weights 1/(1+e^-1), e^-1/(1+e^-1)."""
    for tr in route_trace.read_all(FIXTURE):
        logits = route_trace.logits_for_ids(tr.ids, tr.experts)
        ids, w = oracle.top2_f32(logits)
        assert np.array_equal(ids, tr.ids)
        np.testing.assert_allclose(w[:, 0], 1 / (1 + np.exp(-1.0)), rtol=1e-6)
        np.testing.assert_allclose(w[:, 1], np.exp(-1.0) / (1 + np.exp(-1.0)), rtol=1e-6)
    with pytest.raises(ValueError):
        route_trace.logits_for_ids(np.zeros((4, 3), np.int32), 8)
