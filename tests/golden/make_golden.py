"""Writes tests/golden/paged_attention_v2_cases.npz: the oracle's outputs for the
reference's deterministic-pattern attention cases (tests/golden_cases.py).

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent / "oracle"))

import oracle  # noqa: E402
from golden_cases import GOLDEN_PATH, REFERENCE_CASES  # noqa: E402


def main():
    out = {}
    for name, make in sorted(REFERENCE_CASES.items()):
        c = make()
        out[name] = oracle.paged_attention(c["q"], c["k"], c["v"], c["tables"], c["lens"],
                                           c["num_seqs"], c["num_heads"], c["num_kv_heads"],
                                           c["head_dim"], c["block_size"], c["max_blocks"],
                                           c["scale"])
    np.savez_compressed(GOLDEN_PATH, **out)
    print(GOLDEN_PATH, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
