"""Writes the small fixtures under tests/golden/.

zigzag_kat.json: the known-answer data of the reference's zig-zag unit tests
(hxy0118/fa4-cp tests/test_zigzag.py:21-78), transcribed as plain lists: shard row lists of
test_zigzag_pairs_early_and_late (cp=4, n=32), the half_indices(8) split, get_half_index on
cu=[0,4,12] and cu//2, and zigzag_shard_varlen(cp=2, full_cu=[0,8,24]) -> local_cu.

c4_lengths.json: the packed-varlen benchmark lengths (8 sequences, multiples of 8 in
[1024, 16384], total <= 65536, seed 0) as drawn by the oracle's varlen_lengths.

    python tests/golden/make_golden.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def main():
    from oracle.ring_oracle import varlen_lengths

    kat = {
        "source": "hxy0118/fa4-cp tests/test_zigzag.py:21-78",
        "pairs_early_late": {"cp_size": 4, "n": 32, "rows": {
            "0": [0, 1, 2, 3, 28, 29, 30, 31],
            "1": [4, 5, 6, 7, 24, 25, 26, 27],
            "2": [8, 9, 10, 11, 20, 21, 22, 23],
            "3": [12, 13, 14, 15, 16, 17, 18, 19]}},
        "each_rank_2h": {"cp_size": 4, "n": 64, "rows_per_rank": 16},
        "roundtrip_cp_sizes": [1, 2, 4, 8],
        "half_indices": {"local_len": 8, "first": [0, 1, 2, 3], "second": [4, 5, 6, 7]},
        "get_half_index": {"cu": [0, 4, 12], "front": [0, 1, 4, 5, 6, 7],
                           "back": [2, 3, 8, 9, 10, 11], "half_cu": [0, 2, 6]},
        "shard_varlen": {"cp_size": 2, "full_cu": [0, 8, 24], "local_cu": [0, 4, 12],
                         "local_rows": 12},
    }
    with open(os.path.join(HERE, "zigzag_kat.json"), "w") as f:
        json.dump(kat, f, indent=1)
    with open(os.path.join(HERE, "c4_lengths.json"), "w") as f:
        json.dump({"seed": 0, "lengths": varlen_lengths(0)}, f)


if __name__ == "__main__":
    main()
