"""Writes ``topk_pinned.npz``: the router input the reference's kernel check pins, and the
routing its rule gives, computed here in float64.

The input is the one ``fixed_case`` of tests/python/kernels/moe/test_topk_softmax.py:104-157
builds - ``torch.randn(4, 128)`` from a generator seeded 20240704, times 0.5, row 0's first
three scores set to 10, 5, 5 (an exact tie between picks two and three), rounded to bf16 - and
the expected routing follows that check's statement of the rule: softmax in float64, picks by
descending probability with equal ones in ascending id, renormalised over the picks with an
FP32-epsilon floor. Only torch's own generator is used; no reference code is imported.
"""

from pathlib import Path

import numpy as np
import torch

EXPERTS, TOP, ROWS = 128, 8, 4
FLT_EPSILON = float(np.finfo(np.float32).eps)


def main():
    generator = torch.Generator().manual_seed(20240704)
    scores = torch.randn(ROWS, EXPERTS, generator=generator) * 0.5
    scores[0, 0] = 10.0
    scores[0, 1] = 5.0
    scores[0, 2] = 5.0
    scores = scores.to(torch.bfloat16)
    bits = scores.view(torch.int16).numpy().view(np.uint16).copy()
    exact = scores.double().numpy()

    maximum = exact.max(axis=1, keepdims=True)
    probabilities = np.exp(exact - maximum)
    probabilities /= probabilities.sum(axis=1, keepdims=True)
    ids = np.empty((ROWS, TOP), dtype=np.int32)
    weights = np.empty((ROWS, TOP), dtype=np.float64)
    for row in range(ROWS):
        order = sorted(range(EXPERTS), key=lambda e: (-probabilities[row, e], e))[:TOP]
        ids[row] = order
        picked = probabilities[row, order]
        weights[row] = picked / max(picked.sum(), FLT_EPSILON)
    np.savez(Path(__file__).with_name("topk_pinned.npz"), scores_bf16=bits, ids=ids, weights=weights)


if __name__ == "__main__":
    main()
