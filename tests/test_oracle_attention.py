"""The attention oracle is pinned before anything is compared with it.

  * bit-identical to the reference kernel's own output (the golden fixtures
    were written by the reference build, tests/golden/make_golden.py) and,
    where the reference library is built here, on fresh random shapes;
  * within 1e-5 of a float64 closed-form softmax attention;
  * the closed form itself is checked to catch planted mistakes (wrong
    scale, wrong GQA head mapping, dropped causal mask, K/V swapped).
"""

import numpy as np
import pytest

from helpers import load_golden, sha256
from oracle import attention as oa
from oracle import packing as op

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

CASES = ["fp32_mha_decode", "gqa_prefill", "gqa_decode", "mixed_small", "masked_rows", "empty_context"]


def golden_inputs(name):
    g = load_golden(name)
    if "query" not in g:  # regenerated from the seed
        case = make_golden.fp32_mha_decode_case(0)
        assert sha256(case["query"], case["key_cache"], case["value_cache"]) == str(g["input_sha256"])
        g.update({k: case[k] for k in ("query", "key_cache", "value_cache", "gather_slots", "mask")})
    return g


def f64_from_flat(g):
    """Closed form on the gathered context of a flat reference call."""
    q = g["query"][0]  # [H_q, T, D]
    k_rows = g["key_cache"][0].reshape(-1, g["key_cache"].shape[3], g["key_cache"].shape[4])
    v_rows = g["value_cache"][0].reshape(-1, g["value_cache"].shape[3], g["value_cache"].shape[4])
    slots = g["gather_slots"].astype(np.int64)
    keys = np.transpose(k_rows[slots], (1, 0, 2))  # [H_kv, C, D]
    values = np.transpose(v_rows[slots], (1, 0, 2))
    return oa.attention_f64(q, keys, values, g["mask"][0, 0].astype(bool), float(g["scale"]))


@pytest.mark.parametrize("name", CASES)
def test_oracle_bit_identical_to_reference_output(name):
    g = golden_inputs(name)
    out = oa.paged_attention(g["query"], g["key_cache"], g["value_cache"], 0, g["gather_slots"], g["mask"],
                             float(g["scale"]))
    assert out.shape == g["expected"].shape
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_float64_closed_form(name):
    g = golden_inputs(name)
    out = oa.paged_attention(g["query"], g["key_cache"], g["value_cache"], 0, g["gather_slots"], g["mask"],
                             float(g["scale"]))
    ref = f64_from_flat(g)
    assert np.max(np.abs(out[0] - ref), initial=0.0) < 1e-5


def test_special_cases_give_zeros():
    g = golden_inputs("masked_rows")
    assert np.all(g["expected"][0, 1] == 0) and np.all(g["expected"][0, 4] == 0)
    g = golden_inputs("empty_context")
    assert np.all(g["expected"] == 0)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_bit_identical_on_random_shapes(seed):
    if not oa.reference_available():
        pytest.skip("reference kernel not built here (oracle/_ref)")
    rng = np.random.default_rng(seed)
    hkv = int(rng.integers(1, 4))
    hq = hkv * int(rng.integers(1, 4))
    d = int(rng.choice([4, 8, 16, 32]))
    bs = int(rng.choice([1, 2, 4, 16]))
    b = int(rng.integers(1, 5))
    counts = [int(x) for x in rng.integers(1, 6, size=b)]
    starts = [int(x) for x in rng.integers(0, 20, size=b)]
    case = make_golden.paged_case(100 + seed, hq, hkv, d, bs, starts, counts, scale=float(rng.uniform(0.1, 1.0)))
    args = (case["query"], case["key_cache"], case["value_cache"], 0, case["gather_slots"], case["mask"],
            float(case["scale"]))
    a = oa.paged_attention(*args, kind="oracle")
    r = oa.paged_attention(*args, kind="reference")
    assert np.array_equal(a.view(np.uint32), r.view(np.uint32))


def test_per_sequence_driver_equals_flat_call():
    g = golden_inputs("mixed_small")
    flat = oa.paged_attention(g["query"], g["key_cache"], g["value_cache"], 0, g["gather_slots"], g["mask"],
                              float(g["scale"]))[0]
    per, secs = oa.paged_attention_per_sequence(g["query"][0], g["key_cache"], g["value_cache"], 0,
                                                g["starts"], g["counts"], g["gather_slots"], float(g["scale"]))
    assert secs >= 0.0
    assert np.array_equal(flat.view(np.uint32), per.view(np.uint32))


def test_per_sequence_driver_runs_reference_kernel_too():
    if not oa.reference_available():
        pytest.skip("reference kernel not built here (oracle/_ref)")
    g = golden_inputs("gqa_prefill")
    a, _ = oa.paged_attention_per_sequence(g["query"][0], g["key_cache"], g["value_cache"], 0, g["starts"],
                                           g["counts"], g["gather_slots"], float(g["scale"]), kind="oracle")
    r, _ = oa.paged_attention_per_sequence(g["query"][0], g["key_cache"], g["value_cache"], 0, g["starts"],
                                           g["counts"], g["gather_slots"], float(g["scale"]), kind="reference")
    assert np.array_equal(a.view(np.uint32), r.view(np.uint32))


# ---- the closed form catches plausible mistakes ------------------------

def _planted(g, mistake):
    q = g["query"][0]
    k_rows = g["key_cache"][0].reshape(-1, g["key_cache"].shape[3], g["key_cache"].shape[4])
    v_rows = g["value_cache"][0].reshape(-1, g["value_cache"].shape[3], g["value_cache"].shape[4])
    slots = g["gather_slots"].astype(np.int64)
    keys = np.transpose(k_rows[slots], (1, 0, 2))
    values = np.transpose(v_rows[slots], (1, 0, 2))
    mask = g["mask"][0, 0].astype(bool)
    scale = float(g["scale"])
    if mistake == "scale":
        scale *= 1.25
    elif mistake == "gqa_modulo":  # h % H_kv instead of h // group
        hq, hkv = q.shape[0], keys.shape[0]
        order = [h % hkv for h in range(hq)]
        keys = keys[order]
        values = values[order]
        keys = np.repeat(keys[:, None], 1, axis=1)[:, 0]
        return _f64_per_head(q, keys, values, mask, scale)
    elif mistake == "no_causal":
        qi = op.sequence_index(list(g["counts"]))
        ci = op.sequence_index(list(g["starts"] + g["counts"]))
        mask = ci[None, :] == qi[:, None]
    elif mistake == "kv_swapped":
        keys, values = values, keys
    return oa.attention_f64(q, keys, values, mask, scale)


def _f64_per_head(q, keys, values, mask, scale):
    hq = q.shape[0]
    out = np.zeros((q.shape[1], hq, q.shape[2]))
    for h in range(hq):
        out[:, h] = oa.attention_f64(q[h : h + 1], keys[h : h + 1], values[h : h + 1], mask, scale)[:, 0]
    return out


@pytest.mark.parametrize("mistake", ["scale", "gqa_modulo", "no_causal", "kv_swapped"])
def test_closed_form_rejects_planted_mistakes(mistake):
    g = golden_inputs("gqa_prefill")
    wrong = _planted(g, mistake)
    assert np.max(np.abs(g["expected"][0] - wrong)) > 1e-3
