"""The torch custom-op seam (torch.ops.rwkv7mi.*) on the CPU: every schema is
registered, in-place arguments carry alias annotations, CPU tensors are
refused with RuntimeError (no CPU fallback) and the fake kernels give output
shapes under FakeTensorMode without running anything."""
from __future__ import annotations

import pytest
import torch


def test_every_op_is_registered_with_its_schema():
    import rwkv7mi  # noqa: F401
    from rwkv7mi.ops import SCHEMAS

    for name, schema in SCHEMAS.items():
        op = getattr(torch.ops.rwkv7mi, name).default
        assert str(op._schema).startswith(f"rwkv7mi::{name}("), name
        mutated = [a.name for a in op._schema.arguments if a.alias_info is not None and a.alias_info.is_write]
        assert bool(mutated) == name.endswith("_") or name == "mm8_matmul_out", (name, mutated)


def test_inplace_marks():
    import rwkv7mi  # noqa: F401

    def writes(op):
        return [a.name for a in op.default._schema.arguments if a.alias_info is not None and a.alias_info.is_write]

    assert writes(torch.ops.rwkv7mi.chunk_scan_) == ["state", "y"]
    assert writes(torch.ops.rwkv7mi.fused_recurrent_update_) == ["state", "out"]
    assert writes(torch.ops.rwkv7mi.attn_norm_mix6_) == ["previous", "out"]
    assert writes(torch.ops.rwkv7mi.mm8_matmul_out) == ["out"]


def test_cpu_tensors_are_refused():
    import rwkv7mi  # noqa: F401

    x = torch.zeros(1, 4, 2, 64)
    st = torch.zeros(1, 2, 64, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        torch.ops.rwkv7mi.chunk_scan(x, x, x, x, x, x, st, 0)


def test_fake_kernels_give_shapes():
    import rwkv7mi  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        r = torch.empty(2, 32, 3, 64, dtype=torch.float16)
        st = torch.empty(2, 3, 64, 64)
        y, s = torch.ops.rwkv7mi.chunk_scan(r, r.float(), r, r, r, r, st, 0)
        assert y.shape == r.shape and s.shape == st.shape
        x = torch.empty(5, 256, dtype=torch.float16)
        w = torch.empty(256, 512, dtype=torch.uint8)
        m = torch.empty(512, dtype=torch.float16)
        yy = torch.ops.rwkv7mi.mm8_matmul(x, w, m, m, torch.empty(256, 1, dtype=torch.float16),
                                          torch.empty(256, 1, dtype=torch.float16))
        assert yy.shape == (5, 512)
        outs = torch.ops.rwkv7mi.seq_shift_mix(torch.empty(2, 7, 64), torch.empty(2, 64), [torch.empty(64)] * 3)
        assert len(outs) == 4 and outs[-1].shape == (2, 64)
