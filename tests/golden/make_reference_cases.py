"""Write tests/golden/reference_cases.json: the known answers that UniCache's
own tests pin for the physical KV-cache path, transcribed as data (inputs and
expected outputs) from tests/test_physical.py of the reference, plus the
budget arithmetic of the benchmark configurations (tensor_backend.py:199-210
applied to BASELINE configs 3 and 4).  Run: python tests/golden/make_reference_cases.py"""

import json
import os

CASES = {
    # test_physical.py:1195-1215 -- key = arange(8*2*4).reshape(8, 2, 4)
    "h2o_select_per_kv_head": {
        "tokens": 8, "kv_heads": 2, "head_dim": 4,
        "scores": [[9.0, 8.0, 5.0, 4.0, 3.0, 2.0, 0.0, 0.0],
                   [0.0, 8.0, 1.0, 1.0, 1.0, 9.0, 0.0, 0.0]],
        "target_tokens": 4, "recent_tokens": 2,
        "expected_ids": [[0, 1, 6, 7], [1, 5, 6, 7]],
    },
    # test_physical.py:1021-1053 -- native layout of a 2-bit, G=64 cache
    "native_layout": {
        "tokens": 128, "kv_heads": 2, "head_dim": 64, "bits": 2, "group_size": 64, "residual_length": 0,
        "key_code": [2, 64, 8], "key_scale": [2, 64, 2], "value_code": [2, 128, 4], "value_scale": [2, 128, 1],
        "stats_dtype": "float16",
    },
    # test_physical.py:1070-1097 -- the residual grows to avoid a partial group
    "residual_expansion": {
        "tokens": 320, "kv_heads": 4, "head_dim": 128, "bits": 2, "group_size": 128, "residual_length": 32,
        "quantized_tokens": 256, "residual_tokens": 64,
    },
    # test_physical.py:1099-1132 -- monotonic precision and H2O budget
    "monotonic": {
        "tokens": 64, "kv_heads": 2, "head_dim": 16,
        "kivi": {"bits": 4, "group_size": 8, "residual_length": 8,
                 "repack_down": [2, 16, True], "repack_up": [4, 8, False], "shortfall_events": 1},
        "h2o": {"target_tokens": 16, "recent_tokens": 4,
                "requests": [[8, 2, 8, 8], [16, 4, 8, 8]], "shortfall_tokens": 8},
    },
    # tensor_backend.py:199-210 at a 20% budget for the segments of configs 3 and 4
    "h2o_budget_20pct": [[256, 51, 13], [3840, 768, 192], [4096, 819, 205], [8192, 1638, 410]],
}

if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_cases.json")
    with open(path, "w") as f:
        json.dump(CASES, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", path)
