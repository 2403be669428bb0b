"""Write the packer golden vectors tests/golden/quant_packers.npz.

What they pin: the exact bytes and scales of the three weight packers on the
hot path -- the MM8 affine packer (rwkv7_hf/native_quant_mm8.py:62-97), the
MM4 affine packer (rwkv7_hf/native_quant_mm4.py:77-105) and the symmetric
group-W4 packer (rwkv7_hf/sm70_quant.py:502-519).  Their invariants (every
row/column reaching 0 and 255, reconstruction bounds) leave the order of the
two normalisations and the rounding details open; these vectors do not.

The outputs come from the reference implementation itself
(rwkv-rs/hf-adapter 0.8.1), imported from /root/reference in the build
container only (pure-torch CPU functions) and never shipped.  Inputs are
seeded normal weights (N(0, 0.02)) plus a few edge matrices: a constant row
and column (the eps clamp), an all-zero group and half-step values (the
round-half-to-even of the W4 packer).

Layout of the npz: each input matrix under ``affine__<dtype>_<name>__W`` (MM8
and MM4 share them) or ``w4g__<dtype>_<name>__W``, in the case's dtype, and
each output under ``<packer>__<dtype>_<name>__<reference output name>``.

Run: python tests/golden/make_quant_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "quant_packers.npz"

# [in, out] for the affine packers; both branch orders (in > out, in <= out)
AFFINE_SHAPES = [(40, 24), (24, 40), (3, 5), (5, 3), (33, 33), (256, 128), (128, 256)]
MM4_ODD = [(24, 41), (41, 23), (7, 5)]  # odd out-features: the reference pads one column
# [out, in] with in divisible by the group
W4_CASES = [((24, 256), 128), ((5, 384), 128), ((16, 128), 128), ((8, 512), 256), ((3, 256), 256)]
DTYPES = {"f16": torch.float16, "f32": torch.float32}


def _weights(shape, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * 0.02).astype(np.float32)


def _edge_affine():
    w = _weights((12, 10), 7)
    w[3, :] = 0.125  # constant row
    w[:, 6] = -0.0625  # constant column
    return w


def _edge_w4():
    w = _weights((6, 256), 9)
    w[1, :128] = 0.0  # an all-zero group: scale clamps to 1e-6
    w[2, :128] = np.arange(128, dtype=np.float32) % 14 - 6.5  # k + 0.5 for k in -7..6
    w[2, 0] = 7.0  # max |w| 7 -> scale exactly 1, so the k + 0.5 quotients are exact ties
    w[3, 128:] = np.linspace(-0.5, 0.5, 128, dtype=np.float32)
    return w


def main():
    sys.path.insert(0, "/root/reference")
    from rwkv7_hf.native_quant_mm4 import quantize_mm4
    from rwkv7_hf.native_quant_mm8 import quantize_mm8
    from rwkv7_hf.sm70_quant import quantize_w4_groupwise

    out: dict[str, np.ndarray] = {}

    def put(key, t):
        out[key] = t.detach().cpu().numpy() if torch.is_tensor(t) else np.asarray(t)

    affine = [(f"{i}x{o}", _weights((i, o), 100 + i * 7 + o)) for i, o in AFFINE_SHAPES]
    affine.append(("edge12x10", _edge_affine()))
    odd = [(f"{i}x{o}", _weights((i, o), 200 + i * 7 + o)) for i, o in MM4_ODD]
    for dn, dt in DTYPES.items():
        for name, w in affine + odd:  # one input per matrix, shared by the two affine packers
            put(f"affine__{dn}_{name}__W", torch.tensor(w, dtype=dt))
        for name, w in affine:
            W = torch.tensor(w, dtype=dt)
            key = f"mm8__{dn}_{name}"
            for nm, t in zip(("w_u8", "mx", "rx", "my", "ry"), quantize_mm8(W)):
                put(f"{key}__{nm}", t)
        for name, w in affine + odd:
            W = torch.tensor(w, dtype=dt)
            key = f"mm4__{dn}_{name}"
            packed, mx, rx, my, ry, m_orig, m_pad = quantize_mm4(W)
            for nm, t in (("packed", packed), ("mx", mx), ("rx", rx), ("my", my), ("ry", ry)):
                put(f"{key}__{nm}", t)
            put(f"{key}__m", np.array([m_orig, m_pad], np.int64))
        w4 = [(f"{o}x{i}_g{g}", _weights((o, i), 300 + o * 3 + i + g), g) for (o, i), g in W4_CASES]
        w4.append(("edge6x256_g128", _edge_w4(), 128))
        for name, w, g in w4:
            W = torch.tensor(w, dtype=dt)
            key = f"w4g__{dn}_{name}"
            put(key + "__W", W)
            packed, scales, k = quantize_w4_groupwise(W, group_size=g)
            put(f"{key}__packed", packed)
            put(f"{key}__scales", scales)
            put(f"{key}__group", np.array([g, k], np.int64))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {sum(1 for k in out if k.endswith(('__w_u8', '__packed')))} cases, "
          f"{OUT.stat().st_size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
