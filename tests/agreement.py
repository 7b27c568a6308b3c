"""Top-1 agreement of device tokens with the oracle's logits (the parity.rs protocol of
family/mistral/generation/tests.rs:375-416: teacher-forced steps, >= 99 % agreement).

A step whose device token is not the oracle's argmax still agrees when the oracle's top two
logits are within NEAR_TIE of the logit scale (max |logit|, at least 1): the FP16 roundings of
two implementations may legitimately order such a pair differently. Such steps are counted
and reported, so a test can bound how many it accepted that way.
"""
from __future__ import annotations

import numpy as np

NEAR_TIE = 1e-3


def top1_agreement(tokens, logits, near_tie=NEAR_TIE):
    """Returns (agreeing steps, near ties among them, steps)."""
    agree = ties = steps = 0
    for t, lg in zip(tokens, logits):
        steps += 1
        lg = np.asarray(lg, np.float64)
        if int(t) == int(np.argmax(lg)):
            agree += 1
            continue
        s = np.sort(lg)
        if s[-1] - s[-2] <= near_tie * max(float(np.abs(lg).max()), 1.0):
            agree += 1
            ties += 1
    return agree, ties, steps


def assert_agreement(tokens, logits, what, min_frac=0.99, max_ties=1, near_tie=NEAR_TIE):
    agree, ties, steps = top1_agreement(tokens, logits, near_tie)
    print(f"{what}: top-1 agreement {agree}/{steps}, {ties} of them near ties", flush=True)
    assert agree >= min_frac * steps, (what, agree, steps)
    assert ties <= max_ties, (what, ties)
