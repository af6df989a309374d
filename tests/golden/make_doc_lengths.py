"""Write tests/golden/doc_lengths_pt.json: document lengths for the bench's real-distribution varlen leg.

The reference's bench (scripts/bench.py:84-111, --doc-lengths) fills each training window of
``seq_len`` tokens with documents whose lengths are drawn, with replacement, from the 100,000
Portuguese-corpus document lengths in data/sample_pt/doc_lengths.json, the last one truncated so the
window is exactly full (sore/train/text_sample.py:56-74). This script draws 8 windows of 4,096
tokens (32,768 tokens, BASELINE config 3's total) that way at seed 2026 and stores the lengths, so
the bench and the tests never read the reference at run time.

Run from the repository root with the reference checked out at /root/reference:
    python tests/golden/make_doc_lengths.py
"""
import json
import os
import sys

import numpy as np

SRC = "/root/reference/data/sample_pt/doc_lengths.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "doc_lengths_pt.json")
SEED, WINDOW, WINDOWS = 2026, 4096, 8


def fill_window(pool: np.ndarray, total: int, rng: np.random.Generator) -> list[int]:
    """Lengths drawn with replacement from `pool` (in batches sized by the pool mean) until they add up
    to `total`; the document that crosses the end is cut there."""
    out, filled = [], 0
    while filled < total:
        batch = rng.choice(pool, size=max(1, (total - filled) // int(pool.mean()) + 1))
        for n in batch.tolist():
            n = min(int(n), total - filled)
            out.append(n)
            filled += n
            if filled == total:
                break
    return out


def main() -> int:
    with open(SRC) as f:
        pool = np.asarray(json.load(f)["lengths"], dtype=np.int64)
    if pool.size == 0 or pool.min() < 1:
        raise SystemExit("the length pool must hold positive integers")
    rng = np.random.default_rng(SEED)
    windows = [fill_window(pool, WINDOW, rng) for _ in range(WINDOWS)]
    rec = {
        "source": "data/sample_pt/doc_lengths.json of the reference (100,000 document lengths, Qwen3.5 tokens)",
        "source_stats": {"n": int(pool.size), "mean": float(pool.mean()), "median": float(np.median(pool)),
                         "max": int(pool.max())},
        "seed": SEED, "window": WINDOW, "windows": windows,
    }
    with open(OUT, "w") as f:
        json.dump(rec, f, indent=1)
    flat = [n for w in windows for n in w]
    print(f"wrote {OUT}: {len(flat)} documents, median {np.median(flat):.0f}, max {max(flat)}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
