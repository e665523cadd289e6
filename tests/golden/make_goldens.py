"""Write the page-pooling known answers of the reference's own test.

The values are the literals of ``tests/test_core.py:68-76`` in the LeanSelect
repository (``test_page_pool_uses_overlapping_five_atom_window``): pooling
``arange(15)`` atoms over a 256-token sequence gives pages ``[3, 7, 11, 14]``;
a single hot atom 19 of 31 over a 512-token sequence lights pages 4 and 5.
"""
import json
from pathlib import Path

CASES = [
    {"atoms": list(range(15)), "seq_len": 256, "block_size": 64, "kernel_stride": 16,
     "expected": [3.0, 7.0, 11.0, 14.0]},
    {"atoms": [1.0 if i == 19 else 0.0 for i in range(31)], "seq_len": 512, "block_size": 64,
     "kernel_stride": 16, "expected_nonzero_pages": [4, 5]},
]

if __name__ == "__main__":
    out = Path(__file__).with_name("pool_pages.json")
    out.write_text(json.dumps({"source": "tests/test_core.py:68-76", "cases": CASES}, indent=1))
    print(out)
