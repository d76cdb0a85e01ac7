"""Writes the golden fixtures of tests/golden/ from data the reference's own tests hold.

tau_known_answer.json: the additive-shard cosine test of the reference
(tests/test_parallelism.py:34-44): two rows of 4-element fp32 vectors, threshold 0.5, split
into two shards whose {dot, |old|^2, |new|^2} partial sums are added; the expected decision
is the textbook cosine (computed here in fp64 from the vectors, not from the formula under
test).
"""
import json
import math
import os

OLD = [[1.0, 2.0, -3.0, 4.0], [1.0, 0.0, 1.0, 0.0]]
NEW = [[1.5, 1.0, -2.0, 5.0], [-1.0, 0.0, -1.0, 0.0]]
TAU = 0.5


def main():
    stats = []
    expected = []
    for o, n in zip(OLD, NEW):
        s = [0.0, 0.0, 0.0]
        for lo, hi in ((0, 2), (2, 4)):  # two shards, as the reference test chunks dim -1 in 2
            s[0] += sum(a * b for a, b in zip(o[lo:hi], n[lo:hi]))
            s[1] += sum(a * a for a in o[lo:hi])
            s[2] += sum(b * b for b in n[lo:hi])
        stats.append(s)
        cos = sum(a * b for a, b in zip(o, n)) / math.sqrt(sum(a * a for a in o)) / math.sqrt(sum(b * b for b in n))
        expected.append(cos < TAU)
    out = dict(source="reference tests/test_parallelism.py:34-44", old=OLD, new=NEW, threshold=TAU,
               stats=stats, expected_mask=expected)
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tau_known_answer.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
