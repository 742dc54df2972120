"""Writes `reference_vectors.json`: the literal input/output vectors the reference engine's own
tests hold for this path, transcribed as data (no reference code is imported or run).

Sources (reference repository, `seed_tests/`):
- `test_seed_parity.py:117-130`   MXFP4 hand vector (0x21, 0x73, 0x89 at scales 128 / 125)
- `test_graph_mtp.py:305-318`     `_accept_len` batched case -> [3, 2, 1, 0]
- `test_graph_mtp.py:321-332`     `_fixed_prefix_pack_index` cases at width 4
- `test_mtp_serve.py:216-231`     `_commit_limit` batched case -> [1, 1, 1, 0, 0]
- `test_mtp.py:272-281`           `greedy_accept_length` full / none / partial -> 3 / 0 / 2
- `test_router_fused.py:43-51`    router test shapes (t, experts_out, top_k)
- `test_mxfp4_fused_gemv.py:212-222` the fused-MoE small shapes
  (tokens, experts, hidden, intermediate, top_k)

Run: `python tests/golden/make_reference_vectors.py` (rewrites the JSON beside it).
"""

import json
from pathlib import Path

VECTORS = {
    "mxfp4_hand": {
        "packed_prefix": [0x21, 0x73, 0x89],
        "packed_len": 16,
        "scale_128_first6": [1.0, 2.0, 3.0, 12.0, -1.0, -0.0],
        "scale_125_index3": 1.5,
    },
    "accept_len": {
        "draft": [[5, 6, 7], [5, 6, 7], [5, 9, 7], [1, 2, 3]],
        "step_argmax": [[5, 6, 7, 99], [5, 6, 9, 99], [5, 2, 3, 99], [9, 2, 3, 99]],
        "want": [3, 2, 1, 0],
    },
    "pack_index": {
        "width": 4,
        "cases": [
            {"lengths": [1, 3, 2], "cu": [0, 1, 4, 6], "live": [0, 4, 5, 6, 8, 9]},
            {"lengths": [1, 1, 1], "cu": [0, 1, 2, 3], "live": [0, 4, 8]},
            {"lengths": [4, 4, 4], "cu": [0, 4, 8, 12], "live": list(range(12))},
        ],
    },
    "commit_limit": {
        "step_argmax": [[5, 6, 7], [5, 6, 7], [5, 6, 7], [9, 2, 3], [5, 6, 7]],
        "accept": [2, 2, 1, 0, 2],
        "budget": [9, 2, 9, 9, 1],
        "stops": [[6, -1], [-1, -1], [7, -1], [9, 2], [-1, -1]],
        "want": [1, 1, 1, 0, 0],
    },
    "greedy_accept_length": [
        {"draft": [5, 6, 7], "argmax": [5, 6, 7], "want": 3},
        {"draft": [5, 6, 7], "argmax": [9, 6, 7], "want": 0},
        {"draft": [5, 6, 7], "argmax": [5, 6, 9], "want": 2},
    ],
    "router_shapes": [[1, 4, 1], [5, 8, 2], [3, 512, 10], [4, 17, 3]],
    "moe_small_shapes": [[1, 8, 128, 64, 3], [4, 8, 128, 64, 3], [6, 16, 96, 32, 4], [3, 5, 64, 32, 5]],
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_vectors.json")
    out.write_text(json.dumps(VECTORS, indent=1) + "\n")
    print(f"wrote {out}")
