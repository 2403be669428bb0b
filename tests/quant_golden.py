"""Reader for tests/golden/quant_packers.npz (written by
tests/golden/make_quant_golden.py from the reference's own packers)."""
from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "golden" / "quant_packers.npz"


@lru_cache(maxsize=1)
def _data() -> dict:
    with np.load(PATH) as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


def cases(packer: str) -> list[str]:
    """Case names ("f16_40x24", ...) held for one packer ("mm8", "mm4", "w4g")."""
    marker = {"mm8": "__w_u8", "mm4": "__packed", "w4g": "__packed"}[packer]
    pre = packer + "__"
    return sorted(k[len(pre):-len(marker)] for k in _data() if k.startswith(pre) and k.endswith(marker))


def case(packer: str, name: str) -> dict:
    """Input ``W`` and the reference outputs of one case."""
    d = _data()
    src = "affine" if packer in ("mm8", "mm4") else packer
    out = {"W": d[f"{src}__{name}__W"]}
    pre = f"{packer}__{name}__"
    out.update({k[len(pre):]: v for k, v in d.items() if k.startswith(pre)})
    return out


def bits(a: np.ndarray) -> np.ndarray:
    """The raw bit pattern of a float array, for bit-exact comparisons."""
    a = np.ascontiguousarray(a)
    return a.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]) if a.dtype.kind == "f" else a
