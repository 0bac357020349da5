"""Writes tests/golden/kat.json: the known-answer vectors of the reference's own
tests for the routing path, as data (inputs and expected outputs).

Each entry names the reference test file:line it comes from. The values are
transcribed from those tests; nothing here imports or runs reference code.
Regenerate with `python tests/golden/make_golden.py`.
"""
from __future__ import annotations

import json
from pathlib import Path

NAN = "nan"
INF = "inf"
NINF = "-inf"


def main() -> None:
    kats = {
        "dense_gemm_2x2": {
            "source": "tests/operator_api_tests.cpp:516-531; tests/correctness_framework_tests.cpp:158-164",
            "a": [[1.0, 2.0], [3.0, 4.0]],
            "b": [[5.0, 6.0], [7.0, 8.0]],
            "c": [[19.0, 22.0], [43.0, 50.0]],
        },
        "topk_gate_3x4": {
            "source": "tests/operator_api_tests.cpp:626-660",
            "logits": [[1.0, 3.0, 3.0, 2.0], [NAN, NAN, NAN, NAN], [INF, INF, NINF, 0.0]],
            "ids": [[1, 2], [0, 1], [0, 1]],
            "weights": [[0.5, 0.5], [0.5, 0.5], [0.5, 0.5]],
        },
        "topk_all_nan_1x3": {
            "source": "tests/correctness_framework_tests.cpp:166-172",
            "logits": [[NAN, NAN, NAN]],
            "ids": [[0, 1]],
            "weights": [[0.5, 0.5]],
        },
        "topk_infinity_1x3": {
            "source": "tests/correctness_framework_tests.cpp:173-176",
            "logits": [[INF, 2.0, -1.0]],
            "ids": [[0, 1]],
            "weights": [[1.0, 0.0]],
        },
        "histogram_reset": {
            "source": "tests/operator_api_tests.cpp:662-684",
            "ids": [0, 1, 1, 1],
            "experts": 2,
            "stale_counts": [99, 99],
            "counts": [1, 3],
            "zero_route_counts": [0, 0],
        },
        "histogram_half_split": {
            "source": "tests/operator_api_tests.cpp:706-731",
            "route_pairs": [8192, 32768],
            "pattern": "route & 1",
            "experts": 2,
        },
        "exclusive_scan_mod5": {
            "source": "tests/operator_api_tests.cpp:323-346",
            "experts": [1, 31, 32, 33, 63, 64],
            "counts_rule": "counts[i] = i % 5",
        },
        "exclusive_scan_four_byte_aligned": {
            "source": "tests/operator_api_tests.cpp:364-393",
            "experts": 33,
            "counts_rule": "counts[i] = i % 7",
        },
        "exclusive_scan_int32_max": {
            "source": "tests/operator_api_tests.cpp:395-412",
            "experts": 64,
            "counts_first": 2147483647,
            "offsets_after_first": 2147483647,
        },
        "fused_histogram_scan_round_robin": {
            "source": "tests/operator_api_tests.cpp:442-491",
            "cases": [[0, 1], [1, 8], [257, 33], [4096, 64], [4097, 64]],
            "ids_rule": "ids[r] = r % experts",
        },
        "routing_framework": {
            "source": "tests/correctness_framework_tests.cpp:181-192",
            "ids": [0, 1, 0, 1],
            "experts": 2,
            "counts": [2, 2],
            "offsets": [0, 2, 4],
            "x": [[1.0, 2.0], [3.0, 4.0]],
            "route_pos": [0, 2, 1, 3],
            "sorted_route": [0, 2, 1, 3],
            "x_permuted": [[1.0, 2.0], [3.0, 4.0], [1.0, 2.0], [3.0, 4.0]],
            "top_k": 2,
        },
        "permute_workspace_reset": {
            "source": "tests/operator_api_tests.cpp:734-804",
            "x": [[1.0, 2.0], [3.0, 4.0]],
            "ids": [0, 1, 0, 1],
            "offsets": [0, 2, 4],
            "stale_cursors": [99, 99],
            "final_cursors": [2, 2],
            "top_k": 2,
            "experts": 2,
        },
        "permute_duplicate_ids_unaligned": {
            "source": "tests/operator_api_tests.cpp:806-871",
            "x": [[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]],
            "ids": [0, 0, 1, 1],
            "offsets": [0, 2, 4],
            "top_k": 2,
            "experts": 2,
            "pointer_offset_floats": 1,
        },
        "grouped_unpermute_framework": {
            "source": "tests/correctness_framework_tests.cpp:194-200 (inputs; the reference "
                      "checks only finiteness, y_permuted and y are the hand-computed closed form)",
            "x_permuted": [[1.0, 2.0], [3.0, 4.0], [1.0, 2.0], [3.0, 4.0]],
            "weights": [[[1.0, 0.0], [0.0, 1.0]], [[2.0, 0.0], [0.0, 2.0]]],
            "offsets": [0, 2, 4],
            "y_permuted": [[1.0, 2.0], [3.0, 4.0], [2.0, 4.0], [6.0, 8.0]],
            "route_pos": [0, 2, 1, 3],
            "route_weights": [0.5, 0.5, 0.5, 0.5],
            "y": [[1.5, 3.0], [4.5, 6.0]],
        },
        "unpermute_weighted": {
            "source": "tests/correctness_tests.cpp:252-283",
            "rows": 4,
            "width": 8,
            "row_rule": "y_permuted[r, :] = r + 1",
            "route_weights": [0.25, 0.75, 0.4, 0.6],
            "route_pos": [2, 0, 3, 1],
            "y": [1.5, 2.8],
            "atol": 1e-6,
        },
        "zero_size_contract": {
            "source": "tests/correctness_framework_tests.cpp:236-272",
            "dense_k0": {"m": 2, "n": 2, "k": 0, "c": [0.0, 0.0, 0.0, 0.0]},
            "grouped_k0": {"experts": 1, "hidden": 0, "output": 2, "offsets": [0, 2],
                           "y": [0.0, 0.0, 0.0, 0.0]},
        },
        "route_trace_fixture": {
            "source": "configs/workloads/synthetic_fixture.rrtrace (format: adapter_utils.h:269-322)",
            "schema": "raggedroute.route_trace.v1",
            "trace_id": "synthetic_fixture_t8_e8_top2",
            "source_kind": "synthetic_fixture",
            "tokens": 8, "experts": 8, "top_k": 2,
            "frames": {
                "balanced": [0, 1, 2, 3, 4, 5, 6, 7, 1, 2, 3, 4, 5, 6, 7, 0],
                "skewed": [0, 1, 0, 2, 0, 3, 0, 4, 0, 5, 0, 6, 0, 7, 0, 1],
                "shifted": [7, 6, 6, 5, 5, 4, 4, 3, 3, 2, 2, 1, 1, 0, 0, 7],
            },
        },
    }
    path = Path(__file__).with_name("kat.json")
    path.write_text(json.dumps(kats, indent=1, sort_keys=True) + "\n")
    print(f"wrote {path}")
    # The same fixture as a text trace, frames in the file's order (data, for the
    # native reader's tests).
    fx = kats["route_trace_fixture"]
    lines = [fx["schema"], fx["trace_id"], fx["source_kind"],
             f'{fx["tokens"]} {fx["experts"]} {fx["top_k"]} {len(fx["frames"])}']
    for name in ("balanced", "skewed", "shifted"):
        lines.append(name + " " + " ".join(str(v) for v in fx["frames"][name]))
    trace = Path(__file__).with_name("synthetic_fixture.rrtrace")
    trace.write_text("\n".join(lines) + "\n")
    print(f"wrote {trace}")


if __name__ == "__main__":
    main()
