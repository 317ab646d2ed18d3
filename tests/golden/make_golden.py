"""Writes the golden fixtures for paged decode attention (run once; commit the .npz).

Inputs are regenerated from seeds by tests/golden/cases.py (so the fixtures
stay small); the expected outputs are computed here by fp64
torch.nn.functional.scaled_dot_product_attention on the contiguous K/V the
pool was filled from -- a closed form that shares no code with the oracle or
the kernels. A hash of every input's bytes is stored with the outputs so a
test can tell that it regenerated the same inputs.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from cases import CASES, build  # noqa: E402


def input_digest(case) -> str:
    h = hashlib.sha256()
    for t in (case["q"], case["k_cache"], case["v_cache"]):
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    h.update(np.asarray(case["lens"], dtype=np.int64).tobytes())
    for row in case["tables"]:
        h.update(np.asarray(row, dtype=np.int64).tobytes())
    return h.hexdigest()


def closed_form(case) -> np.ndarray:
    outs = []
    for s, n in enumerate(case["lens"]):
        q = case["q"][s].double().unsqueeze(0).unsqueeze(2)           # [1, Hq, 1, D]
        k = case["k_flat"][s].double().permute(1, 0, 2).unsqueeze(0)  # [1, Hkv, L, D]
        v = case["v_flat"][s].double().permute(1, 0, 2).unsqueeze(0)
        o = F.scaled_dot_product_attention(q, k, v, scale=case["scale"], enable_gqa=True)
        outs.append(o[0, :, 0, :].numpy())
    return np.stack(outs)


def main():
    for name in CASES:
        case = build(name)
        out = closed_form(case)
        np.savez_compressed(HERE / f"{name}.npz", expected=out.astype(np.float64),
                            digest=np.array(input_digest(case)))
        print(f"{name}: {out.shape} digest {input_digest(case)[:16]}")


if __name__ == "__main__":
    main()
