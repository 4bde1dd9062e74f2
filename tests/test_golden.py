"""Oracle vs golden vectors written by the reference's own functions.

``tests/golden/make_golden.py`` ran the reference's selector and predictor
(loaded from its source text, CPU) and saved inputs and outputs. Here the
oracle replays the same inputs.

Selector: teacher-forced per layer (the oracle gets the reference's ledger
state of the previous layer), so every layer checks the layer's math alone.
Priorities agree to float32 rounding (different reduction order) and the
selection must be identical except inside classes of exactly equal
priority at the cut, where torch.topk's order is unspecified and the oracle
keeps the lower index.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import pooling as OP
from oracle import selector as OS

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    path = GOLDEN / name
    if not path.exists():
        pytest.skip(f"{name} not generated")
    return np.load(path)


def _state_from(rec, l):
    return {
        OS.STATE_KEY: rec["debt"][l - 1],
        OS.PENDING_KEY: rec["arrival"][l - 1],
        OS.PENDING_LAYER_KEY: l - 1,
        OS.SERVICE_KEY: {"layer_idx": l - 1, "identity_observed": True,
                         "pair_service_fraction": rec["service"][l - 1]},
    }


def _same_modulo_ties(ours, ref, prio_ref, count):
    """True when the two selections differ only inside an exact tie class."""
    if np.array_equal(ours, ref):
        return True, 0
    rows = np.argwhere((ours != ref).any(-1))
    for idx in map(tuple, rows):
        c = int(count[idx])
        pr = prio_ref[idx]
        if c == 0:
            return False, 0
        cut = np.sort(pr)[::-1][c - 1]
        diff = np.flatnonzero(ours[idx] != ref[idx])
        if not np.all(pr[diff] == cut):
            return False, 0
        if ours[idx].sum() != ref[idx].sum():
            return False, 0
    return True, len(rows)


def _replay(rec, layers, *, hint=None):
    tie_rows = 0
    for l in range(layers):
        st = {} if l == 0 else _state_from(rec, l)
        prot = rec["protected"][l].astype(bool)
        sel, info = OS.cosa_select(rec["score"][l], rec["value"][l], rec["cap"][l], layer_idx=l, state=st,
                                   protected=prot if prot.any() else None, max_capacity_hint=hint)
        ref_prio = rec["priority"][l]
        fin = ref_prio < 1e30
        np.testing.assert_allclose(info["priority"][fin], ref_prio[fin], rtol=2e-6, atol=1e-30)
        assert np.array_equal(info["priority"][~fin], ref_prio[~fin])
        ok, n = _same_modulo_ties(sel, rec["selected"][l].astype(bool), ref_prio, info["count"])
        assert ok, f"layer {l}: selection differs outside exact ties"
        tie_rows += n
        for key in ("debt", "arrival"):
            np.testing.assert_allclose(info[key].reshape(-1), rec[key][l].reshape(-1), rtol=2e-6, atol=1e-9)
        if n == 0:
            np.testing.assert_array_equal(info["service"].reshape(-1), rec["service"][l].reshape(-1))
    return tie_rows


def test_selector_check_protocol_goldens():
    g = _load("selector_check.npz")
    ties = 0
    for K in (1, 2, 7, 8, 31):
        for p in (0, 1):
            pre = f"K{K}_p{p}_"
            rec = {k[len(pre):]: g[k] for k in g.files if k.startswith(pre)}
            ties += _replay(rec, rec["score"].shape[0])
            assert bool(rec["terminal_nonempty"]) and bool(rec["second_finalize_empty"])
    assert ties <= 3  # exact ties at saturated priorities are rare but real


def test_selector_c1_chain_goldens():
    g = _load("selector_c1.npz")
    rec = {k: g[k] for k in g.files}
    _replay(rec, rec["score"].shape[0], hint=int(130 * 0.25) + 1)
    # the ledger accrued debt in the chain, so the debt-priority path is covered
    assert (rec["debt"][1:] > 0).any()


def test_terminal_settlement_matches_golden():
    g = _load("selector_c1.npz")
    L = g["score"].shape[0]
    st = _state_from({k: g[k] for k in g.files}, L)
    out = OS.finalize(st)
    assert out and OS.finalize(st) == {}
    np.testing.assert_allclose(st[OS.STATE_KEY].reshape(-1), g["terminal_debt"].reshape(-1), rtol=2e-6, atol=1e-9)


def test_predict_attention_goldens_bit_exact_after_bf16():
    g = _load("predict.npz")
    n = len([f for f in g.files if f.startswith("prob") and "dtype" not in f])
    loose = 0
    for i in range(n):
        q, k, ref = g[f"q{i}"], g[f"k{i}"], g[f"prob{i}"]
        prob, _, _ = OP.pooled_prob(q, k, bf16=True)
        # the reference ran under CPU autocast, whose softmax output is bf16
        assert np.array_equal(OP.bf16_round(prob), ref), f"case {i}"
        wrong, _, _ = OP.pooled_prob(q, k, bf16=False)
        loose += int(not np.array_equal(OP.bf16_round(wrong), ref))
    assert loose >= 1  # dropping the bf16 logit rounding is detected
