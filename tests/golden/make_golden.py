"""Writes tests/golden/c1_expected.npz: the CPU oracle's scores and argmax for
config C1 plus the sha256 of the generated inputs (so a change of torch's RNG
or of the generator is detected instead of silently changing the fixture).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE))

from c1_inputs import digest, make_c1  # noqa: E402
from oracle import maxsim_oracle  # noqa: E402


def main() -> None:
    q, d, qlen, dlen = make_c1(0)
    scores, argmax = maxsim_oracle.padded_forward(q.numpy(), d.numpy(), qlen.numpy(), dlen.numpy())
    np.savez_compressed(
        HERE / "c1_expected.npz",
        scores=scores,
        argmax=argmax,
        input_sha256=np.array(digest(q, d, qlen, dlen)),
        torch_version=np.array(torch.__version__),
    )
    print(f"wrote c1_expected.npz: scores {scores.shape}, argmax {argmax.shape}")


if __name__ == "__main__":
    main()
