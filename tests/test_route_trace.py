"""Route traces on the host: the native `.rrtrace` reader (rr_route_trace_read)
against the reference's fixture (configs/workloads/synthetic_fixture.rrtrace,
transcribed into tests/golden) and planted format errors, and the writer's
round trip. CPU only.
"""
from __future__ import annotations

import ctypes
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
    (lambda s: s.replace("raggedroute.route_trace.v1", "raggedroute.route_trace.v2"), "line 1"),
    (lambda s: s.replace("synthetic_fixture_t8_e8_top2", "bad id!"), "line 2"),
    (lambda s: s.replace("\nsynthetic_fixture\n", "\nsynthetic\n"), "line 3"),
    (lambda s: s.replace("8 8 2 3", "0 8 2 3"), "shape out of range"),
    (lambda s: s.replace("8 8 2 3", "8 0 2 3"), "shape out of range"),
    (lambda s: s.replace("8 8 2 3", "8 1025 2 3"), "shape out of range"),
    (lambda s: s.replace("8 8 2 3", "8 8 9 3"), "shape out of range"),
    (lambda s: s.replace("8 8 2 3", "8 8 2 0"), "shape out of range"),
    (lambda s: s.replace("8 8 2 3", "8 8 2"), "four integers"),
    # (a fifth word is the first frame's id, as in the reference's stream read)
    (lambda s: s.replace("8 8 2 3", "8 8 2 3 1"), "non-integer"),
    (lambda s: s.replace("8 8 2 3", "8 8 2 x"), "four integers"),
    # a word is a whole decimal integer (the reference's stream extraction
    # would read 2 and then take x as the next word): a deliberate difference
    (lambda s: s.replace("balanced 0 1", "balanced 0 1x"), "non-integer"),
    (lambda s: s.replace("skewed", "balanced"), "share a frame id"),
    (lambda s: s.replace("skewed", "sk/ewed"), "frame id"),
    (lambda s: s.replace("balanced 0 1", "balanced 0 8"), "outside"),
    (lambda s: s.replace("balanced 0 1", "balanced -1 1"), "outside"),
    (lambda s: s.replace("balanced 0 1", "balanced 0 x"), "non-integer"),
    (lambda s: s.replace("balanced 0 1", "balanced 0 1.0"), "non-integer"),
    (lambda s: s.replace("balanced 0 1", "balanced 1 1"), "twice"),
    (lambda s: s.replace("shifted 7 6", "shifted 7 7"), "twice"),
    (lambda s: s + "extra\n", "follows the last frame"),
    (lambda s: s.rsplit(" ", 1)[0] + "\n", "ends early"),
    (lambda s: "", "line 1"),
])
def test_reader_rejects_planted_errors(tmp_path, mutate, message):
    bad = mutate(GOOD)
    assert bad != GOOD
    with pytest.raises(ValueError, match=message):
        route_trace.read(_write(tmp_path, bad), 0)


@pytest.mark.parametrize("mutate", [
    lambda s: s.replace("8 8 2 3\n", "8 8\n2 3\n"),     # the shape over two lines
    lambda s: s.replace("8 8 2 3\n", "8\n8\n2\n3\n"),  # one number a line
    lambda s: s.replace("8 8 2 3\n", "8 8 2 3 "),        # the first record on line 4
    lambda s: s.replace("\n", "\r\n"),                   # CRLF line ends
])
def test_reader_accepts_the_shape_wherever_lines_break(tmp_path, mutate):
    """After the three header lines the shape is read as four words, as the
    reference reads it with stream extraction (reference
    include/raggedroute/benchmark/adapter_utils.h:276-281)."""
    text = mutate(GOOD)
    assert text != GOOD
    for index in range(3):
        got, want = route_trace.read(_write(tmp_path, text), index), route_trace.read(FIXTURE, index)
        assert (got.frame_id, got.tokens, got.experts, got.top_k) == (want.frame_id, 8, 8, 2)
        assert np.array_equal(got.ids, want.ids)


def test_reader_accepts_layout_variants(tmp_path):
    """CRLF line ends, records wrapped over several lines and a missing final
    newline read the same ids as the fixture."""
    variants = [GOOD.replace("\n", "\r\n"), GOOD.replace(" 4 5 ", "\n4 5\n "), GOOD.rstrip("\n")]
    for i, text in enumerate(variants):
        path = _write(tmp_path, text, f"v{i}.rrtrace")
        for index in range(3):
            assert np.array_equal(route_trace.read(path, index).ids, route_trace.read(FIXTURE, index).ids)


def test_reader_argument_errors(tmp_path):
    with pytest.raises(ValueError, match="cannot be opened"):
        route_trace.read(tmp_path / "missing.rrtrace", 0)
    with pytest.raises(ValueError, match="past the last frame"):
        route_trace.read(FIXTURE, 3)
    with pytest.raises(ValueError, match="frame index >= 0"):
        route_trace.read(FIXTURE, -1)


def test_error_in_a_later_frame_leaves_the_buffer_untouched(tmp_path):
    bad = _write(tmp_path, GOOD.replace("shifted 7 6", "shifted 7 7"))
    info = rr.RouteTraceInfo()
    buf = np.full(16, -5, np.int32)
    st = rr.lib.rr_route_trace_read(str(bad).encode(), 0, ctypes.byref(info), buf.ctypes.data, 16)
    assert st.code == rr.StatusCode.kInvalidArgument and (buf == -5).all()


def test_write_reproduces_the_reference_fixture(tmp_path, kat):
    """The writer lays the fixture's frames out byte for byte as the
    reference's normalised fixture file, and the reader returns them."""
    raw = kat.raw["route_trace_fixture"]
    frames = {f: np.array(raw["frames"][f]).reshape(8, 2) for f in FRAMES}
    out = tmp_path / "fixture.rrtrace"
    text = route_trace.write(out, raw["trace_id"], raw["source_kind"], raw["experts"], frames)
    assert text == GOOD and out.read_text() == GOOD
    assert route_trace.read(out, 1).ids.reshape(-1).tolist() == raw["frames"]["skewed"]


@pytest.mark.parametrize("top_k,experts", [(1, 1), (4, 64), (8, 1024)])
def test_write_read_round_trip(tmp_path, top_k, experts):
    from raggedroute_amd import workloads
    frames = {f"f{i}.{d}": workloads.topk_route_ids(37, top_k, experts, d, seed=i)
              for i, d in enumerate(("uniform", "zipf", "round_robin"))}
    path = tmp_path / "rt.rrtrace"
    route_trace.write(path, "gen_trace-1", "captured", experts, frames)
    back = route_trace.read_all(path)
    assert [t.frame_id for t in back] == list(frames)
    for tr, ids in zip(back, frames.values()):
        assert (tr.tokens, tr.top_k, tr.experts, tr.source_kind) == (37, top_k, experts, "captured")
        assert np.array_equal(tr.ids, ids)


@pytest.mark.parametrize("call,message", [
    (lambda w: w("a b", "captured", 8, {"f": np.zeros((2, 1), int)}), "trace id"),
    (lambda w: w("t", "lab", 8, {"f": np.zeros((2, 1), int)}), "source kind"),
    (lambda w: w("t", "captured", 8, {}), "at least one frame"),
    (lambda w: w("t", "captured", 2000, {"f": np.zeros((2, 1), int)}), "outside"),
    (lambda w: w("t", "captured", 8, {"f/1": np.zeros((2, 1), int)}), "frame id"),
    (lambda w: w("t", "captured", 8, {"a": np.zeros((2, 1), int), "b": np.zeros((3, 1), int)}), "one"),
    (lambda w: w("t", "captured", 8, {"f": np.full((2, 1), 8)}), "in \\[0, 8\\)"),
    (lambda w: w("t", "captured", 8, {"f": np.array([[1, 1]])}), "twice"),
    (lambda w: w("t", "captured", 2, {"f": np.array([[0, 1, 2]])}), "in \\[0, 2\\)"),
])
def test_writer_refuses_what_the_reader_would(tmp_path, call, message):
    path = tmp_path / "never.rrtrace"
    with pytest.raises(ValueError, match=message):
        call(lambda *a: route_trace.write(path, *a))
    assert not path.exists()


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
