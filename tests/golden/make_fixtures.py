"""Writes the JSON fixtures under tests/golden/.

The reference stores no golden outputs (all its cases are seeded random), so
the fixtures are the fixed data its tests and docs do hold, transcribed here:

* reshape_and_cache_doc_example.json — the worked example of
  doc/op_docs/reshape_and_cache.md:137-146 (4 tokens, 2 kv heads, head 8,
  4 blocks of 2 slots, slot_mapping [0, 1, 3, 6]) with the (block, offset)
  each token must land in, from the doc's rule block = slot / block_size,
  offset = slot % block_size (reshape_and_cache.md:13-22).
* reference_cases.json — the shapes and fixed length vectors of the
  reference's C++ test cases:
  test/zoo/teco/flash_attention/test_case/{0..5}.prototxt,
  test/zoo/teco/rms_norm/test_case/case_{0..7}.prototxt,
  test/zoo/teco/reshape_and_cache/test_case/case_{0,1,2}.prototxt,
  test/zoo/teco/causal_conv1d/test_case/case_{0,1}.prototxt,
  and the python API tests python_api_test/test_*.py.
  The GPU parity tests replay these shapes with seeded inputs.

Run:  python tests/golden/make_fixtures.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

DOC_EXAMPLE = {
    "num_tokens": 4, "num_kv_heads": 2, "head_size": 8,
    "num_blocks": 4, "block_size": 2,
    "slot_mapping": [0, 1, 3, 6],
    # token t -> (block, offset)
    "expected_placement": [[0, 0], [0, 1], [1, 1], [3, 0]],
}

REFERENCE_CASES = {
    "flash_attention": [
        # name, H, Hkv, D, block_size, num_blocks, q_lens, kv_lens, block_table dims
        {"name": "fa_case0", "H": 32, "Hkv": 8, "D": 128, "bs": 32, "num_blocks": 8,
         "q_lens": [256], "kv_lens": [256], "bt_cols": 8},
        {"name": "fa_case1", "H": 32, "Hkv": 8, "D": 128, "bs": 32, "num_blocks": 256,
         "q_lens": [1, 256, 128], "kv_lens": [511, 257, 511], "bt_cols": 16},
        {"name": "fa_case2", "H": 16, "Hkv": 2, "D": 128, "bs": 32, "num_blocks": 256,
         "q_lens": [1, 256, 128], "kv_lens": [512, 256, 512], "bt_cols": 16},
        {"name": "fa_case3", "H": 16, "Hkv": 4, "D": 128, "bs": 32, "num_blocks": 256,
         "q_lens": [1, 256, 128], "kv_lens": [512, 256, 512], "bt_cols": 16},
        {"name": "fa_case4", "H": 16, "Hkv": 8, "D": 64, "bs": 32, "num_blocks": 256,
         "q_lens": [1, 256, 128], "kv_lens": [512, 256, 512], "bt_cols": 16},
        {"name": "fa_case5", "H": 2, "Hkv": 1, "D": 128, "bs": 32, "num_blocks": 35845,
         "q_lens": [22], "kv_lens": [22], "bt_cols": 16},
        # python_api_test/test_flash_attention.py:258-355 (block 32, 64 blocks)
        {"name": "py_prefill_2x64_128", "H": 8, "Hkv": 4, "D": 128, "bs": 32,
         "num_blocks": 64, "q_lens": [64, 128], "kv_lens": [64, 128], "bt_cols": 4},
        {"name": "py_decode_2x128", "H": 8, "Hkv": 4, "D": 128, "bs": 32, "num_blocks": 64,
         "q_lens": [1, 1], "kv_lens": [128, 64], "bt_cols": 4},
        {"name": "py_chunked_2b_32x64", "H": 8, "Hkv": 4, "D": 128, "bs": 32,
         "num_blocks": 64, "q_lens": [32, 16], "kv_lens": [64, 32], "bt_cols": 2},
        {"name": "py_gqa_2q_1kv_decode_2b", "H": 2, "Hkv": 1, "D": 128, "bs": 32,
         "num_blocks": 64, "q_lens": [1, 1], "kv_lens": [64, 128], "bt_cols": 4},
        {"name": "py_mix_decode_prefill", "H": 8, "Hkv": 4, "D": 128, "bs": 32,
         "num_blocks": 64, "q_lens": [1, 32], "kv_lens": [128, 64], "bt_cols": 4},
    ],
    "rms_norm": [
        # test/zoo/teco/rms_norm/test_case/case_{0..7}: 64 rows; pure and add
        {"tokens": 64, "hidden": 4096, "eps": 1e-6, "residual": False},
        {"tokens": 64, "hidden": 4096, "eps": 1e-6, "residual": True},
        {"tokens": 64, "hidden": 2048, "eps": 1e-5, "residual": False},
        {"tokens": 64, "hidden": 2048, "eps": 1e-5, "residual": True},
        {"tokens": 64, "hidden": 1536, "eps": 1e-6, "residual": False},
        {"tokens": 64, "hidden": 1536, "eps": 1e-6, "residual": True},
        {"tokens": 64, "hidden": 128, "eps": 1e-6, "residual": False},
        {"tokens": 64, "hidden": 128, "eps": 1e-5, "residual": False},
    ],
    "reshape_and_cache": [
        # case_{0,1,2}: 512 tokens, 64 blocks x 16 slots, head 128
        {"tokens": 512, "kv_heads": 8, "head": 128, "num_blocks": 64, "block_size": 16},
        {"tokens": 512, "kv_heads": 4, "head": 128, "num_blocks": 64, "block_size": 16},
        {"tokens": 512, "kv_heads": 2, "head": 128, "num_blocks": 64, "block_size": 16},
    ],
    "causal_conv1d": [
        # C++ case_0 / case_1 and python_api_test/test_causal_conv1d.py:158-196
        {"dim": 2048, "seq_lens": [8], "cache_indices": [0], "has_init": [0],
         "num_entries": 1, "pad_slot_id": -1},
        {"dim": 2048, "seq_lens": [6, 10], "cache_indices": [0, 1], "has_init": [0, 0],
         "num_entries": 2, "pad_slot_id": -1},
        {"dim": 1280, "seq_lens": [256, 256], "cache_indices": [0, 1], "has_init": [0, 0],
         "num_entries": 2, "pad_slot_id": -1},
        {"dim": 2048, "seq_lens": [8], "cache_indices": [0], "has_init": [1],
         "num_entries": 1, "pad_slot_id": -1},
        {"dim": 256, "seq_lens": [6, 6], "cache_indices": [-1, 2], "has_init": [0, 1],
         "num_entries": 4, "pad_slot_id": -1},
    ],
}


def main():
    with open(os.path.join(HERE, "reshape_and_cache_doc_example.json"), "w") as f:
        json.dump(DOC_EXAMPLE, f, indent=1)
    with open(os.path.join(HERE, "reference_cases.json"), "w") as f:
        json.dump(REFERENCE_CASES, f, indent=1)


if __name__ == "__main__":
    main()
