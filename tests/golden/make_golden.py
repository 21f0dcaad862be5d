"""Write tests/golden/sdpa_known_answer.npz (run once, in a tree that has the reference).

The reference's only stored attention known answer is the masked SDPA
snapshot tests/model/snapshots/test_scaled_dot_product_attention.npz, an
output of shape (4, 12, 64) for inputs its tests regenerate from torch seeds
(tests/model/conftest.py:88-116): q = randn(4, 12, 64) after manual_seed(1),
k = randn(4, 16, 64) after seed 2, v = randn(4, 16, 64) after seed 3 and
mask = randn(4, 12, 16) > 0.5 after seed 5. This script reads that snapshot
as data (numpy, allow_pickle=False), regenerates the inputs the same way and
stores inputs and expected output together, so the fixture does not depend on
torch's RNG at test time.

    python tests/golden/make_golden.py /root/reference
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main(reference_root: str) -> None:
    snapshot = os.path.join(reference_root, "tests", "model", "snapshots",
                            "test_scaled_dot_product_attention.npz")
    with np.load(snapshot, allow_pickle=False) as data:
        expected = np.array(data["array"])
    torch.manual_seed(1)
    q = torch.randn(4, 12, 64)
    torch.manual_seed(2)
    k = torch.randn(4, 16, 64)
    torch.manual_seed(3)
    v = torch.randn(4, 16, 64)
    torch.manual_seed(5)
    mask = torch.randn(4, 12, 16) > 0.5
    out = os.path.join(HERE, "sdpa_known_answer.npz")
    np.savez_compressed(out, q=q.numpy(), k=k.numpy(), v=v.numpy(),
                        mask=mask.numpy(), expected=expected)
    print(out)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
