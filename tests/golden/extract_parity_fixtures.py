"""Writes tests/golden/parity_dumps/*.json: the JSON documents held by the
reference comparator's unit tests (crates/fish_s2_parity/src/lib.rs:2354-2459).

Run in the build container, where the reference checkout is at
/root/reference; the GPU box and the tests only read the committed JSON.
"""

import json
import os

SRC = "/root/reference/crates/fish_s2_parity/src/lib.rs"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "parity_dumps")
FIXTURES = {
    "slow_ar_single.json": "test_slow_ar_dump_json",
    "slow_ar_sequence.json": "test_slow_ar_sequence_dump_json",
    "slow_ar_full_block.json": "test_slow_ar_full_block_dump_json",
}


def main():
    src = open(SRC).read()
    os.makedirs(OUT, exist_ok=True)
    for name, fn in FIXTURES.items():
        i = src.index(f"fn {fn}() -> &'static str")
        j = src.index('r#"', i) + 3
        doc = json.loads(src[j:src.index('"#', j)])
        with open(os.path.join(OUT, name), "w") as f:
            json.dump(doc, f, indent=2)
        print("wrote", name)


if __name__ == "__main__":
    main()
