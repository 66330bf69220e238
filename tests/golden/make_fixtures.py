"""Write the golden fixtures of this directory.

The numbers are transcribed from the reference's own unit tests (inputs and expected outputs
only); the reference code is neither imported nor run:
  route_metadata_kat.json  tests/ut/modules/mega_moe/test_route.py:402-528
                           (test_async_count_gather_overlaps_permute_and_builds_metadata)
  permute_kat.json         tests/ut/examples/moe/test_native_experts.py:59-80
                           (gather order <-> scatter mapping convention)
Run: python tests/golden/make_fixtures.py
"""
import json
from pathlib import Path

HERE = Path(__file__).resolve().parent

ROUTE_METADATA_KAT = {
    "source": "tests/ut/modules/mega_moe/test_route.py:402-528",
    "ep_size": 2,
    "rank": 1,
    "num_experts": 4,
    "supplied_counts": [5, 6, 7, 8],
    "global_counts": [[1, 2, 3, 4], [5, 6, 7, 8]],
    "expected_received_counts": [[3, 4], [7, 8]],
    "push": {
        "dispatch_src_off": [0, 5, 11, 18],
        "dispatch_target_off": [1, 8, 3, 14],
        "dispatch_size": [5, 6, 7, 8],
        "combine_src_off": [0, 10, 3, 14],
        "combine_target_off": [3, 6, 11, 18],
        "combine_size": [3, 4, 7, 8],
        "group_list": [10, 22],
        "expert_capacity": 22,
    },
    "pull": {
        "dispatch_src_off": [3, 6, 11, 18],
        "dispatch_target_off": [0, 10, 3, 14],
        "dispatch_size": [3, 4, 7, 8],
    },
}

PERMUTE_KAT = {
    "source": "tests/ut/examples/moe/test_native_experts.py:59-80",
    "gather_order": [0, 1, 3, 4, 5, 6, 2],
    "scatter_mapping": [0, 1, 6, 2, 3, 4, 5],
    "note": "one-slot-per-token expert ids whose stable expert sort yields the gather order",
    "topk_ids": [[0], [0], [2], [1], [1], [1], [1]],
    "num_experts": 3,
}


def main() -> None:
    (HERE / "route_metadata_kat.json").write_text(json.dumps(ROUTE_METADATA_KAT, indent=1) + "\n")
    (HERE / "permute_kat.json").write_text(json.dumps(PERMUTE_KAT, indent=1) + "\n")


if __name__ == "__main__":
    main()
