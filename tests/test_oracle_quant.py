"""Pins of the CPU packers / dequant oracles (CPU only).

Bit-exactness of the packers rests on the restatement using the reference's
fp32 op sequence (rwkv7_hf/native_quant_mm8.py:62-97,
rwkv7_hf/sm70_quant.py:502-519, rwkv7_hf/native_quant_mm4.py:77-105).  The
invariants below are consequences of that algorithm that a wrong branch order,
a missing /16 or a wrong rounding mode would break.
"""
from __future__ import annotations

import numpy as np
import pytest


@pytest.mark.parametrize("shape", [(40, 24), (24, 40), (33, 33), (3, 5), (5, 3)])
def test_mm8_every_row_and_column_hits_0_and_255(oracle, shape):
    rng = np.random.default_rng(1)
    W = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    q, *_ = oracle.mm8_pack(W)
    assert q.dtype == np.uint8
    assert (q.min(axis=0) == 0).all() and (q.min(axis=1) == 0).all()
    assert (q.max(axis=0) == 255).all() and (q.max(axis=1) == 255).all()


def test_mm8_branch_order_tall_vs_wide(oracle):
    rng = np.random.default_rng(2)
    tall = (rng.standard_normal((50, 20)) * 0.02).astype(np.float32)
    _, mx, rx, my, ry = oracle.mm8_pack(tall, out_dtype=np.float32)
    np.testing.assert_array_equal(my.reshape(-1), tall.min(axis=1))  # rows first when N > M
    wide = (rng.standard_normal((20, 50)) * 0.02).astype(np.float32)
    _, mx, rx, my, ry = oracle.mm8_pack(wide, out_dtype=np.float32)
    np.testing.assert_array_equal(mx, wide.min(axis=0))  # columns first when N <= M


@pytest.mark.parametrize("shape", [(64, 48), (48, 64)])
def test_mm8_reconstruction_bound(oracle, shape):
    rng = np.random.default_rng(3)
    W = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    q, mx, rx16, my, ry16 = oracle.mm8_pack(W, out_dtype=np.float32)
    deq = oracle.mm8_dequant(q, mx, rx16, my, ry16)
    bound = (np.asarray(ry16, np.float64).reshape(-1, 1) * 16) * (np.asarray(rx16, np.float64).reshape(1, -1) * 16) / 512
    assert (np.abs(deq - W) <= bound * (1 + 1e-5) + 1e-7).all()


def test_mm8_constant_matrix(oracle):
    W = np.full((6, 4), 0.25, np.float32)
    q, mx, rx16, my, ry16 = oracle.mm8_pack(W, out_dtype=np.float32)
    assert (q == 0).all()
    np.testing.assert_array_equal(my.reshape(-1), np.full(6, 0.25, np.float32))
    np.testing.assert_array_equal(mx, np.zeros(4, np.float32))
    np.testing.assert_array_equal(rx16, np.full(4, np.float32(1e-8) / np.float32(16), np.float32))


def test_mm8_gemv_two_forms_agree(oracle):
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((96, 80)) * 0.02).astype(np.float32)
    packed = oracle.mm8_pack(W)
    x = rng.standard_normal((5, 96))
    np.testing.assert_allclose(oracle.mm8_matmul(x, *packed), oracle.mm8_matmul_split(x, *packed),
                               rtol=1e-11, atol=1e-11)




@pytest.mark.parametrize("group", [128, 256])
def test_w4g_kat_shapes_and_invariants(oracle, group):
    # tests/test_sm70_quant.py:118-125: [24, 256] -> packed [24, 128], scales [24, 256/group]
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((24, 256)) * 0.02).astype(np.float32)
    packed, scales, k = oracle.w4g_pack(W, group, out_dtype=np.float32)
    assert packed.shape == (24, 128) and scales.shape == (24, 256 // group) and k == 256
    lo, hi = packed & 15, packed >> 4
    assert lo.min() >= 1 and hi.min() >= 1 and lo.max() <= 15 and hi.max() <= 15
    g = W.reshape(24, 256 // group, group)
    np.testing.assert_array_equal(scales, np.maximum(np.abs(g).max(-1) / np.float32(7), np.float32(1e-6)))
    deq = oracle.w4g_dequant(packed, scales, group)
    s_full = np.repeat(scales.astype(np.float64), group, axis=1)
    assert (np.abs(deq - W) <= s_full / 2 * (1 + 1e-6)).all()
    # the largest-magnitude element of every group lands on +-7
    q = np.empty((24, 256), np.int64)
    q[:, 0::2] = lo.astype(np.int64) - 8
    q[:, 1::2] = hi.astype(np.int64) - 8
    idx = np.abs(g).argmax(-1)
    qg = q.reshape(24, 256 // group, group)
    assert (np.abs(np.take_along_axis(qg, idx[..., None], -1)) == 7).all()


def test_w4g_rounds_half_to_even(oracle):
    # scale = 7/7 = 1 exactly, so w/s is exact and ties are visible
    W = np.zeros((1, 128), np.float32)
    W[0, 0] = 7.0
    W[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 4.5]
    packed, scales, _ = oracle.w4g_pack(W, 128, out_dtype=np.float32)
    assert scales[0, 0] == 1.0
    q = np.empty(128, np.int64)
    q[0::2] = (packed[0] & 15).astype(np.int64) - 8
    q[1::2] = (packed[0] >> 4).astype(np.int64) - 8
    np.testing.assert_array_equal(q[:9], [7, 0, 2, 2, 0, -2, -2, 4, 4])


def test_mm4_invariants(oracle):
    rng = np.random.default_rng(6)
    W = (rng.standard_normal((40, 31)) * 0.02).astype(np.float32)  # odd M is padded to 32
    packed, mx, rx4, my, ry4, m_orig, m_pad = oracle.mm4_pack(W, out_dtype=np.float32)
    assert packed.shape == (40, 16) and m_orig == 31 and m_pad == 32
    u = np.empty((40, 32), np.int64)
    u[:, 0::2] = packed & 15
    u[:, 1::2] = packed >> 4
    assert (u.min(0) == 0).all() and (u.max(1) == 15).all()
    deq = oracle.mm4_dequant(packed, mx, rx4, my, ry4, m_orig)
    bound = (np.asarray(ry4, np.float64).reshape(-1, 1) * 4) * (np.asarray(rx4, np.float64).reshape(1, -1)[:, :31] * 4) / 32
    assert (np.abs(deq - W) <= bound * (1 + 1e-5) + 1e-7).all()


def test_w4a_pack_closed_forms(oracle):
    """The asymmetric (min/max affine) group W4 packer: in every non-constant
    group the minimum maps to 0 and the maximum to 15; a constant group is
    reproduced exactly by its bias; the reconstruction error is at most half a
    step plus the fp16 rounding of scale and bias; a hand-computed known answer
    (a ramp whose step is exactly representable) and a planted mistake (a
    symmetric-style centring) that the bound catches."""
    rng = np.random.default_rng(41)
    O, I, G = 6, 512, 128
    W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    W[2, 128:256] = 0.0125  # a constant group
    packed, sc, bi = oracle.w4a_pack(W, G)
    q = np.empty((O, I), np.uint8)
    q[:, 0::2], q[:, 1::2] = packed & 15, packed >> 4
    qg = q.reshape(O, I // G, G)
    for o in range(O):
        for g in range(I // G):
            grp = W[o, g * G:(g + 1) * G]
            if grp.max() > grp.min():
                assert qg[o, g][grp.argmin()] == 0 and qg[o, g][grp.argmax()] == 15
            else:
                assert (qg[o, g] == 0).all()
    deq = oracle.w4a_dequant(packed, sc, bi, G)
    assert deq[2, 128:256].tolist() == [float(np.float16(0.0125))] * 128
    s32 = np.repeat(((W.reshape(O, -1, G).max(-1) - W.reshape(O, -1, G).min(-1)) / 15), G, axis=1)
    bound = s32 / 2 + 15 * np.abs(s32) * 2.0 ** -11 + np.abs(W).max() * 2.0 ** -11
    assert (np.abs(deq - W) <= bound + 1e-12).all()
    # known answer: w = 0.25 * j - 1 over one group of 128 (j = 0..127 -> q = rint(j * 15 / 127))
    ramp = (0.25 * np.arange(128, dtype=np.float32) - 1.0)[None]
    p2, s2, b2 = oracle.w4a_pack(ramp, 128)
    assert float(b2[0, 0]) == -1.0 and float(s2[0, 0]) == float(np.float16(np.float32(31.75) / np.float32(15)))
    q2 = np.empty(128, np.uint8)
    q2[0::2], q2[1::2] = p2[0] & 15, p2[0] >> 4
    np.testing.assert_array_equal(q2, np.rint(np.arange(128) * (0.25 / np.float32(31.75 / 15))).clip(0, 15))
    # planted: centring each group on 0 instead of its minimum breaks the bound
    planted = (np.clip(np.rint(W.reshape(O, -1, G) / s32.reshape(O, -1, G)[..., :1]), -8, 7)
               * s32.reshape(O, -1, G)[..., :1]).reshape(O, I)
    assert (np.abs(planted - W) > bound).any()


# ---------------------------------------------------------------- reference bytes
# tests/golden/quant_packers.npz holds the reference packers' own outputs
# (rwkv7_hf/native_quant_mm8.py:62-97, native_quant_mm4.py:77-105,
# sm70_quant.py:502-519) on seeded and edge inputs, fp16 and fp32, both branch
# orders, odd MM4 widths and groups 128 / 256.  The oracle must reproduce every
# byte and every scale bit.
import quant_golden as qg  # noqa: E402


def _np_dtype(W):
    return np.float16 if W.dtype == np.float16 else np.float32


@pytest.mark.parametrize("name", qg.cases("mm8"))
def test_mm8_pack_matches_reference_bytes(oracle, name):
    c = qg.case("mm8", name)
    got = oracle.mm8_pack(c["W"].astype(np.float32), out_dtype=_np_dtype(c["W"]))
    for g, key in zip(got, ("w_u8", "mx", "rx", "my", "ry")):
        assert g.shape == c[key].shape, key
        np.testing.assert_array_equal(qg.bits(g), qg.bits(c[key]), err_msg=f"{name} {key}")


@pytest.mark.parametrize("name", qg.cases("mm4"))
def test_mm4_pack_matches_reference_bytes(oracle, name):
    c = qg.case("mm4", name)
    packed, mx, rx, my, ry, m_orig, m_pad = oracle.mm4_pack(c["W"].astype(np.float32), out_dtype=_np_dtype(c["W"]))
    assert [m_orig, m_pad] == c["m"].tolist()
    for g, key in ((packed, "packed"), (mx, "mx"), (rx, "rx"), (my, "my"), (ry, "ry")):
        assert g.shape == c[key].shape, key
        np.testing.assert_array_equal(qg.bits(g), qg.bits(c[key]), err_msg=f"{name} {key}")


@pytest.mark.parametrize("name", qg.cases("w4g"))
def test_w4g_pack_matches_reference_bytes(oracle, name):
    c = qg.case("w4g", name)
    group, k = c["group"].tolist()
    packed, scales, kk = oracle.w4g_pack(c["W"].astype(np.float32), group, out_dtype=_np_dtype(c["W"]))
    assert kk == k
    np.testing.assert_array_equal(packed, c["packed"], err_msg=name)
    np.testing.assert_array_equal(qg.bits(scales), qg.bits(c["scales"]), err_msg=name)


def _affine_pack_planted(W, levels, mistake):
    """numpy fp32 restatement of the affine packers with one planted mistake;
    used only to show that the reference fixtures reject it."""
    w = W.astype(np.float32)
    n, m = w.shape
    rows_first = n > m
    if mistake == "branch":
        rows_first = not rows_first
    if rows_first:
        my = w.min(1, keepdims=True); w = w - my
        mx = w.min(0); w = w - mx
    else:
        mx = w.min(0); w = w - mx
        my = w.min(1, keepdims=True); w = w - my
    eps = np.float32(1e-8)
    if mistake == "ry_before_rx":
        ry = np.maximum(w.max(1, keepdims=True), eps); w = w / ry
        rx = np.maximum(w.max(0), eps); w = w / rx
    else:
        rx = np.maximum(w.max(0), eps); w = w / rx
        ry = np.maximum(w.max(1, keepdims=True), eps); w = w / ry
    if mistake == "round":
        return np.clip(np.rint(w * np.float32(levels)), 0, levels - 1).astype(np.uint8)
    return np.clip(np.floor(w * np.float32(levels)), 0, levels - 1).astype(np.uint8)


def test_mm8_fixtures_reject_planted_packers():
    """The unplanted restatement reproduces the fixtures' bytes; normalising
    rows before columns, swapping the branch order or rounding to nearest each
    changes bytes in most cases (invariant pins alone pass such packers)."""
    names = [n for n in qg.cases("mm8") if "edge" not in n and "33x33" not in n]
    for name in names:
        c = qg.case("mm8", name)
        np.testing.assert_array_equal(_affine_pack_planted(c["W"], 256, None), c["w_u8"])
    for mistake in ("ry_before_rx", "branch", "round"):
        caught = sum(not np.array_equal(_affine_pack_planted(qg.case("mm8", n)["W"], 256, mistake),
                                        qg.case("mm8", n)["w_u8"]) for n in names)
        assert caught >= len(names) - 2, (mistake, caught, len(names))


def test_w4g_fixtures_reject_planted_rounding():
    """Round half away from zero (instead of torch.round's half to even) must
    change the edge case's bytes: its group holds exact k + 0.5 quotients."""
    c = qg.case("w4g", "f32_edge6x256_g128")
    W = c["W"].astype(np.float32)
    s = np.maximum(np.abs(W.reshape(6, 2, 128)).max(-1) / np.float32(7), np.float32(1e-6))
    t = W.reshape(6, 2, 128) / s[..., None]
    for rnd, ok in ((np.rint, True), (lambda x: np.sign(x) * np.floor(np.abs(x) + 0.5), False)):
        q = (np.clip(rnd(t), -7, 7).astype(np.int16) + 8).reshape(6, 256)
        packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
        assert np.array_equal(packed, c["packed"]) == ok
