"""Write ``pack_kats.json``: the reference's known-answer vectors for this path.

Each entry restates, as data, an input and the expected output that one of the
reference's own tests asserts (the source line is kept in ``"source"``).  The
expected words are written out as integers here, not computed by any packer,
so the fixture checks the oracle rather than agreeing with it by construction.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
from pathlib import Path


def main() -> None:
    kats = {
        "pack_2bit_k128": {
            "source": "tests/test_pack.py:26-41",
            "shape": [1, 128],
            "codes_nonone": {"0": 2, "1": 1, "15": 2, "16": 3},
            "default_code": 0,
            "words": [0x80000006, 3, 0, 0, 0, 0, 0, 0],
        },
        "pack_2bit_one_word": {
            "source": "tests/test_pack.py:44-52",
            "codes": [i % 3 for i in range(16)],
        },
        "pack_4bit": {
            "source": "tests/test_pack.py:102-111",
            "shape": [1, 64],
            "codes_nonone": {"0": 10, "1": 3, "7": 15},
            "default_code": 0,
            "word0": 0xF000003A,
        },
        "ternary_gemv_lsb_first": {
            "source": "tests/test_ternary_gemv.py:114-132",
            "n": 2,
            "k": 128,
            "default_code": 1,
            "codes_set": [[0, 0, 2], [1, 1, 0]],
            "alpha": [0.5, 1.25],
            "x": "arange(128)",
            "y": [0.0, -1.25],
        },
        "ternarize_zero_rows": {
            "source": "tests/test_pack.py:95-99",
            "shape": [2, 128],
            "codes": 1,
            "alpha": 0.0,
        },
    }
    # The one-word KAT: codes (i % 3) for i in 0..15, code i in bits 2i..2i+1.
    # Written out term by term: codes 1 at i = 1,4,7,10,13 and 2 at i = 2,5,8,11,14.
    ones = [1, 4, 7, 10, 13]
    twos = [2, 5, 8, 11, 14]
    word = sum(1 << (2 * i) for i in ones) + sum(2 << (2 * i) for i in twos)
    kats["pack_2bit_one_word"]["word"] = word
    out = Path(__file__).with_name("pack_kats.json")
    out.write_text(json.dumps(kats, indent=1, sort_keys=True) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
