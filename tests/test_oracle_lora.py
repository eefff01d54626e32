"""Pin the LoRA oracle to the reference's fixtures (closed forms) and to
torch.nn.functional.linear."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import lora as ol

VECTORS = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _mods(case):
    out = []
    for m in case["modules"]:
        a = np.full((m["rank"], case["in_features"]), m["a_const"])
        b = np.full((m["out_features"], m["rank"]), m["b_const"])
        out.append((m, a, b))
    return out


@pytest.mark.parametrize("case", VECTORS["lora"], ids=lambda c: c["source"][:50])
def test_reference_fixture_per_module(case):
    x = np.array(case["x"])
    for m, a, b in _mods(case):
        w = np.array(m["weight"])
        bias = None if m["bias"] is None else np.array(m["bias"])
        np.testing.assert_allclose(ol.lora_delta(x, a, b, m["scale"]), m["expected_delta"], atol=1e-12)
        np.testing.assert_allclose(ol.lora_linear(x, w, bias, a, b, m["scale"]), m["expected_output"], atol=1e-12)
        np.testing.assert_allclose(ol.merged_linear(x, w, bias, a, b, m["scale"]), m["expected_output"], atol=1e-12)


@pytest.mark.parametrize("case", VECTORS["lora"], ids=lambda c: c["source"][:50])
def test_reference_fixture_packed(case):
    x = np.array(case["x"])
    mods = _mods(case)
    packed = ol.packed_lora_delta(x, [(a, b, m["scale"]) for m, a, b in mods])
    want = np.concatenate([np.array(m["expected_delta"]) for m, _, _ in mods], axis=1)
    np.testing.assert_allclose(packed, want, atol=1e-12)
    a_cat, b_bd = ol.pack_lora([(a, b, m["scale"]) for m, a, b in mods])
    # packed shapes of packed_ops.py:362-375 as the reference tests assert them
    assert a_cat.shape == (sum(m["rank"] for m, _, _ in mods), case["in_features"])
    assert b_bd.shape == (sum(m["out_features"] for m, _, _ in mods), a_cat.shape[0])
    # B_bd is block diagonal: zero outside each module's (rows, rank) block
    assert np.count_nonzero(b_bd) == sum(m["out_features"] * m["rank"] for m, _, _ in mods)


def test_random_against_torch_linear():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 24))
    w = rng.standard_normal((12, 24))
    bias = rng.standard_normal(12)
    a = rng.standard_normal((4, 24))
    b = rng.standard_normal((12, 4))
    s = 1.75
    xt, wt, bt, at, btt = (torch.from_numpy(t) for t in (x, w, bias, a, b))
    want = F.linear(xt, wt, bt) + F.linear(F.linear(xt, at), btt) * s
    np.testing.assert_allclose(ol.lora_linear(x, w, bias, a, b, s), want.numpy(), atol=1e-12)
    np.testing.assert_allclose(ol.merged_linear(x, w, bias, a, b, s), want.numpy(), atol=1e-10)
    # a dropped scale or transposed operand would not pass
    assert not np.allclose(ol.lora_delta(x, a, b, s), ol.lora_delta(x, a, b, 1.0))


def test_multi_adapter_matches_per_adapter_delta():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((9, 16))
    A = rng.standard_normal((3, 4, 16))
    B = rng.standard_normal((3, 10, 4))
    ids = [0, 2, 1, -1, 2, 0, 3, 1, 1]
    got = ol.multi_adapter_delta(x, ids, A, B, 2.0)
    for t, i in enumerate(ids):
        want = ol.lora_delta(x[t:t + 1], A[i], B[i], 2.0)[0] if 0 <= i < 3 else np.zeros(10)
        np.testing.assert_allclose(got[t], want, atol=1e-12)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-8, 8, 10000),
                        [0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.4e38, -3.4e38, 1e-40]])
    want = torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(ol.round_bf16(v), want)
    np.testing.assert_array_equal(ol.round_to(v[:20], "f16"), torch.from_numpy(v[:20]).half().double().numpy())


def test_intermediate_rounding_is_applied_to_down_projection():
    rng = np.random.default_rng(3)
    x, a, b = rng.standard_normal((4, 32)), rng.standard_normal((2, 32)), rng.standard_normal((8, 2))
    down = ol.round_bf16(x @ a.T)
    np.testing.assert_allclose(ol.lora_delta(x, a, b, 2.0, intermediate="bf16"), down @ b.T * 2.0, atol=1e-12)
    assert not np.allclose(ol.lora_delta(x, a, b, 2.0, intermediate="bf16"), ol.lora_delta(x, a, b, 2.0), atol=1e-9)
