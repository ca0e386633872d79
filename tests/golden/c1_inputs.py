"""Seeded generator of configuration C1 (padded rerank, fp32): 8 queries x 16
candidates, Lq = 32, documents padded to Ld = 300 with real lengths uniform in
[64, 300], dim = 128, L2-normalised Gaussian rows.  Pad rows hold garbage on
purpose (they must be ignored).  Shared by make_golden.py and the tests."""

from __future__ import annotations

import hashlib

import numpy as np
import torch
import torch.nn.functional as F

B, C, LQ, LD, DIM = 8, 16, 32, 300, 128


def make_c1(seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, LQ, DIM, generator=g), dim=-1)
    d = F.normalize(torch.randn(B, C, LD, DIM, generator=g), dim=-1)
    qlen = torch.full((B,), LQ, dtype=torch.int32)
    dlen = torch.randint(64, LD + 1, (B, C), generator=g, dtype=torch.int32)
    # garbage beyond the real lengths
    pad = torch.arange(LD)[None, None, :] >= dlen[:, :, None]
    d = d.masked_fill(pad[..., None], 1e4)
    return q, d, qlen, dlen


def digest(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(np.ascontiguousarray(t.numpy()).tobytes())
    return h.hexdigest()
