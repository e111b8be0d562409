"""CPU restatement of the reference's eager attention baseline.

TEST INFRASTRUCTURE ONLY (timed by ``bench.py``'s ``cpu_baseline`` leg).

Follows ``standard_eager_attention`` in benchmark-gb10/run_study.py:304-335, operation by
operation and in the input dtype, as the reference's "eager" method runs it:

1. ``scores = (q @ k^T) * (1/sqrt(D))`` in the input dtype;
2. causal: ``where(triu(ones(S,S), 1), finfo(dtype).min, scores)``;
3. ``softmax(scores, dim=-1, dtype=float32)`` cast back to the input dtype;
4. ``probs @ v``.

This is the *timed CPU baseline*, not the correctness oracle: its matmuls round to
fp16/bf16.  ``eager_attention_per_head`` runs the same math one (b, h) slice at a time so
that long sequences fit in host memory (the score matrix of one head at S=16384 is 512 MiB
in fp16 plus 1 GiB in fp32); results are identical because heads are independent.
"""

from __future__ import annotations

import math


def eager_attention(q, k, v, *, causal: bool, causal_mask=None):
    import torch

    scale = 1.0 / math.sqrt(float(q.shape[-1]))
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        if causal_mask is None:
            s = scores.shape[-1]
            causal_mask = torch.ones((1, 1, s, s), device=scores.device, dtype=torch.bool).triu(1)
        neg = torch.tensor(torch.finfo(scores.dtype).min, dtype=scores.dtype, device=scores.device)
        scores = torch.where(causal_mask, neg, scores)
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, v)


def eager_attention_per_head(q, k, v, *, causal: bool, heads=None):
    """Same math as ``eager_attention`` over a subset of (b, h) slices, one at a time.

    ``heads``: iterable of (b, h) pairs (default: all).  Returns the list of outputs.
    """
    import torch

    b_, h_, s, _ = q.shape
    mask = torch.ones((1, 1, s, s), dtype=torch.bool).triu(1) if causal else None
    pairs = heads if heads is not None else [(b, h) for b in range(b_) for h in range(h_)]
    outs = []
    for b, h in pairs:
        outs.append(eager_attention(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                                    causal=causal, causal_mask=mask))
    return outs
