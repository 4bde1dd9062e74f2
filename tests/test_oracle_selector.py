"""Pins of oracle/selector.py beyond the golden vectors: the reference's
check_selector invariants and closed forms that fix the arithmetic."""
import itertools

import numpy as np
import pytest

from oracle import selector as OS


def _softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


def test_select_top_matches_brute_force_with_lower_index_ties():
    rng = np.random.default_rng(0)
    for K in range(1, 7):
        for _ in range(30):
            prio = rng.integers(0, 3, K).astype(np.float32)  # many exact ties
            for c in range(K + 1):
                got = OS.select_top(prio, np.array(c))
                # brute force: among all subsets of size c, the lexicographically best
                # (sorted priorities descending, then smallest indices)
                best = None
                for sub in itertools.combinations(range(K), c):
                    key = (sorted(prio[list(sub)], reverse=True), [-i for i in sub])
                    if best is None or key > best[0]:
                        best = (key, sub)
                expect = np.zeros(K, bool)
                expect[list(best[1])] = True
                assert np.array_equal(got, expect), (prio, c)


def test_selected_indices_match_torch_topk_on_distinct_priorities():
    """The selector's selected_indices are ``priority.topk(M, sorted=True)``
    (SW:3887-3894); on rows without ties torch's own topk fixes every entry,
    including the order."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    for K in (1, 2, 7, 130, 518, 2072):
        prio = rng.permutation(np.arange(4 * K, dtype=np.float32))[:K] / np.float32(7)
        prio = np.stack([prio, rng.permutation(prio), np.float32(3) - prio])
        for M in sorted({0, 1, K // 4, K // 2 + 1, K}):
            got = OS.selected_indices(prio, M)
            expect = torch.from_numpy(prio).topk(M, dim=-1, sorted=True).indices.numpy()
            assert got.dtype == np.int64 and got.shape == (3, M)
            assert np.array_equal(got, expect), (K, M)


def test_selected_indices_brute_force_with_ties():
    """Descending priority, equal priorities in ascending index (the tie rule
    of the selection); the first c entries are the selected set."""
    rng = np.random.default_rng(12)
    for K in range(1, 9):
        for _ in range(40):
            prio = rng.integers(0, 3, K).astype(np.float32)
            prio[rng.random(K) < 0.1] = np.float32(3.4028235e38)  # protected blocks
            full = OS.selected_indices(prio, K)
            assert full.tolist() == sorted(range(K), key=lambda k: (-float(prio[k]), k))
            for c in range(K + 1):
                sel = np.zeros(K, bool)
                sel[full[:c]] = True
                assert np.array_equal(sel, OS.select_top(prio, np.array(c)))


def test_check_selector_invariants():
    """tests/check_selector.py:44-65 of the reference, on the oracle."""
    rng = np.random.default_rng(20260906)
    active = 0
    for K in (1, 2, 7, 8, 31):
        for protect in (False, True):
            st = {}
            for layer in range(24):
                scores = _softmax(rng.standard_normal((1, 2, 3, K)))
                values = rng.standard_normal((1, 2, K, 13)).astype(np.float32)
                cap = rng.integers(0, K + 1, (1, 2, 3))
                prot = np.zeros((1, 2, 3, K), bool)
                if protect:
                    prot[..., -1] = cap > 0
                sel, info = OS.cosa_select(scores, values, cap, layer_idx=layer, state=st, protected=prot)
                assert np.array_equal(sel.sum(-1), cap)
                assert sel[prot].all()
                assert np.isfinite(st["cosa_value_risk_pair_priority"]).all()
                active += bool((st[OS.STATE_KEY] > 0).any())
            assert OS.finalize(st)
            assert OS.finalize(st) == {}
    assert active > 0


def test_layer0_priority_is_conservative_arrival():
    rng = np.random.default_rng(1)
    s = _softmax(rng.standard_normal((1, 3, 5, 20)))
    v = rng.standard_normal((1, 3, 20, 64)).astype(np.float32)
    sel, info = OS.cosa_select(s, v, np.full((1, 3, 5), 6), layer_idx=0, state={})
    assert not info["gate"]
    A, _, _, _ = OS.conservative_arrival(s, OS.innovation(v), np.full((1, 3, 5), 6))
    assert np.array_equal(info["priority"], A)
    # closed form of the conservative projection on one row
    iota_k = np.repeat(OS.innovation(v), 2, axis=-1)
    risk = s[0, 0, 0].astype(np.float64) * iota_k[0, 0]
    closed = np.clip(risk * 6 / risk.sum(), 0, 1)
    np.testing.assert_allclose(A[0, 0, 0], closed, rtol=1e-5)


def test_uniform_innovation_unsaturated_reduces_to_topk():
    rng = np.random.default_rng(2)
    K = 40
    s = _softmax(0.1 * rng.standard_normal((1, 2, 7, K)))  # flat: cap * share < 1 everywhere
    v = np.zeros((1, 2, K, 64), np.float32)
    v[:, :, 1::2, :] = 1.0  # every pair differs by the same amount
    iota = OS.innovation(v)
    assert np.all(iota == iota.flat[0]) and iota.flat[0] > 0
    cap = np.full((1, 2, 7), 10)
    sel, info = OS.cosa_select(s, v, cap, layer_idx=0, state={})
    assert info["priority"].max() < 1
    assert np.array_equal(sel, OS.select_top(s, cap))


def test_zero_innovation_selects_first_blocks():
    s = _softmax(np.random.default_rng(3).standard_normal((1, 1, 4, 12)))
    v = np.ones((1, 1, 12, 64), np.float32)
    sel, info = OS.cosa_select(s, v, np.full((1, 1, 4), 5), layer_idx=0, state={})
    assert np.all(info["priority"] == 0)
    assert np.array_equal(sel[0, 0], np.tile(np.arange(12) < 5, (4, 1)))


def test_zero_debt_keeps_gate_closed_and_settlement_conserves():
    rng = np.random.default_rng(4)
    K, Q = 16, 6
    st = {}
    for layer in range(3):
        s = _softmax(rng.standard_normal((1, 2, Q, K)))
        v = rng.standard_normal((1, 2, K, 64)).astype(np.float32)
        prev_debt = st.get(OS.STATE_KEY)
        pending = st.get(OS.PENDING_KEY)
        service = None if pending is None else st[OS.SERVICE_KEY]["pair_service_fraction"]
        sel, info = OS.cosa_select(s, v, np.full((1, 2, Q), 5), layer_idx=layer, state=st)
        if layer == 0:
            assert not info["gate"] and np.all(info["debt"] == 0)
        else:
            d0 = np.zeros_like(pending) if prev_debt is None else prev_debt
            # D' - D - A + S - refl == 0 up to one float32 rounding per term
            resid = info["debt"].reshape(d0.shape) - d0 - pending + service - info["reflection"].reshape(d0.shape)
            assert np.abs(resid).max() <= 4 * np.finfo(np.float32).eps
        # service counts every selected child once: sum(service*pair_size*Q) == selected blocks
        ps = np.where(np.arange((K + 1) // 2) == (K + 1) // 2 - 1, 1 + (K % 2 == 0), 2)
        assert np.isclose((info["service"] * ps * Q).sum(), sel.sum())


def test_gate_rule_examples():
    serv = np.array([[[0.5, 0.5]]], np.float32)
    assert OS.service_gate(serv, np.zeros_like(serv))          # nothing wasted
    assert not OS.service_gate(np.zeros_like(serv), np.zeros_like(serv))  # no service at all
    refl = np.array([[[0.5, 0.5]]], np.float32)
    assert not OS.service_gate(serv, refl + 0.1)               # waste exceeds useful repayment


def test_topk_block_mask_sink_and_min_one():
    s = _softmax(np.random.default_rng(5).standard_normal((1, 2, 3, 9)))
    m = OS.topk_block_mask(s, 2, sparse_ratio=0.99)  # int(9*0.01) = 0 -> fill rule keeps 1
    assert np.array_equal(m[..., :9].sum(-1), np.ones((1, 2, 3)))
    assert m[..., 9:].all()
    assert np.array_equal(m[..., :9].argmax(-1), s.argmax(-1))


@pytest.mark.parametrize("official", [True, False])
def test_layer_selection_mixed_tail(official):
    # C1 geometry: 8288 patch tokens -> 130 key blocks, the last holding 32 patch tokens
    s = _softmax(np.random.default_rng(6).standard_normal((1, 2, 65, 130)))
    final, _ = OS.layer_selection(s, mode="topk", sparse_ratio=0.75, patch_tokens=8288, total_tokens=8328,
                                  official_mask=official)
    assert final.shape[-1] == 131 and final[..., 130].all()
    assert final[..., 129].all() == (not official)
    st = {}
    final_v, info = OS.layer_selection(s, mode="vasc", sparse_ratio=0.75, patch_tokens=8288, total_tokens=8328,
                                       official_mask=official, state=st, layer_idx=0,
                                       pooled_value=np.random.default_rng(7).standard_normal((1, 2, 130, 64)))
    assert np.array_equal(final_v[..., :130].sum(-1), final[..., :130].sum(-1))
    if not official:
        assert final_v[..., 129].all()


# ---------------------------------------------------------------- cdf threshold
def _torch_cdf_counts(score, thr, topk=None, eps=1e-5):
    """get_block_mask's cdf steps (SW:1238-1254) and the fill rule
    (utils.py:289) with torch's own sort / cumsum / searchsorted."""
    import torch
    s = torch.from_numpy(score)
    B, H, Q, K = s.shape
    cdf = torch.cumsum(torch.sort(s, dim=-1, descending=True).values, dim=-1)
    t = torch.as_tensor(thr, dtype=torch.float32)
    t = torch.full((H,), float(t)) if t.ndim == 0 else t
    t = (t.view(1, H, 1, 1) + eps).expand(B, -1, Q, 1).contiguous()
    n = torch.searchsorted(cdf, t, right=True).squeeze(-1)
    if topk is not None:
        n = torch.clamp(n, min=topk)
    return torch.where(n == 0, torch.ones_like(n), n).numpy()


@pytest.mark.parametrize("K", [1, 7, 64, 130, 518])
def test_cdf_counts_match_torch_on_dyadic_scores(K):
    """Scores k/1024: every prefix sum is exact in float32 (and float64), so
    torch's scan and the sequential sum agree bit for bit. Thresholds sit
    exactly on prefix sums, just below them and in between."""
    rng = np.random.default_rng(K)
    s = (rng.integers(0, 65, size=(1, 3, 5, K)) / 1024).astype(np.float32)
    cdf = np.cumsum(-np.sort(-s, axis=-1), axis=-1)
    p = float(cdf[0, 0, 0, K // 2])
    picks = [0.0, p, p - 2e-5, p - 5e-6, 0.37, float(cdf.max()) + 1.0]  # p - 5e-6 is kept only through eps
    for thr in picks:
        for topk in (None, 0, max(K // 4, 1)):
            got = OS.cdf_counts(s, thr, topk)
            assert np.array_equal(got, _torch_cdf_counts(s, thr, topk)), (thr, topk)
    per_head = [0.1, 0.25, 0.5]
    assert np.array_equal(OS.cdf_counts(s, per_head), _torch_cdf_counts(s, np.array(per_head, np.float32)))


def test_cdf_counts_sequential_float32_brute_force():
    """Non-dyadic softmax rows: the running sum is the strictly sequential
    float32 one (a loop over the descending row)."""
    rng = np.random.default_rng(11)
    s = _softmax(rng.standard_normal((1, 2, 6, 37)) * 2)
    for thr in (0.3, 0.6, 0.9, 0.99):
        got = OS.cdf_counts(s, thr)
        T = np.float32(np.float32(thr) + np.float32(1e-5))
        for h, q in itertools.product(range(2), range(6)):
            row = np.sort(s[0, h, q])[::-1]
            acc, n = np.float32(0.0), 0
            for v in row:
                acc = np.float32(acc + v)
                if not acc <= T:
                    break
                n += 1
            assert got[0, h, q] == max(n, 1)


def test_cdf_counts_brute_force_on_every_row_kind():
    """Rows that are not softmax rows, against a loop written from the
    definition alone: NaN first, then the values in descending order (-0 and
    +0 equal), a strictly sequential float32 running sum, the count of the
    prefix that stays <= T, then the fill rule. Row kinds: signed scores
    with zeros (the sum falls), NaN and infinities, few distinct values, all
    equal, mostly zero."""
    rng = np.random.default_rng(13)
    K = 300
    rows = [
        (rng.standard_normal(K) * 0.01).astype(np.float32),
        _softmax(rng.standard_normal(K) * 0.5),
        _softmax(np.round(rng.standard_normal(K))),
        np.full(K, 1.0 / K, np.float32),
        np.zeros(K, np.float32),
        _softmax(rng.standard_normal(K) * 0.5),
        _softmax(rng.standard_normal(K) * 0.5),
    ]
    rows[0][rng.random(K) < 0.2] = 0.0
    rows[0][:3] = [-0.0, 0.0, -0.0]
    rows[1][rng.integers(0, K, 2)] = np.nan          # NaN sorts first: the count is 1
    rows[4][rng.integers(0, K, 20)] = rng.random(20).astype(np.float32) / 20
    rows[5][[7, 11]] = [np.inf, -np.inf]
    rows[6][13] = -np.inf                             # last: counted once the sum reaches it
    s = np.stack(rows).reshape(1, 1, len(rows), K)
    for thr in (0.0, 0.02, 0.5, 0.9, 1.0):
        got = OS.cdf_counts(s, thr)
        T = np.float32(np.float32(thr) + np.float32(1e-5))
        for q, row in enumerate(rows):
            order = sorted(range(K), key=lambda i: (not np.isnan(row[i]), -float(row[i]) if not np.isnan(row[i]) else 0.0, i))
            acc, n = np.float32(0.0), 0
            for i in order:
                acc = np.float32(acc + row[i])
                if not acc <= T:
                    break
                n += 1
            assert got[0, 0, q] == max(n, 1), (thr, q)


def test_cdf_counts_closed_forms():
    K = 256
    u = np.full((1, 1, 2, K), 1.0 / K, np.float32)  # cdf[i] = (i+1)/K exactly
    assert (OS.cdf_counts(u, 0.5) == K // 2).all()
    assert (OS.cdf_counts(u, 1.0) == K).all()          # the full sum 1.0 <= 1 + eps
    assert (OS.cdf_counts(u, 0.0) == 1).all()          # nothing fits: fill rule keeps one block
    assert (OS.cdf_counts(u, 0.0, topk=5) == 5).all()  # the ratio budget is a lower bound
    # without the eps, a threshold equal to a prefix sum keeps it anyway (right=True)
    assert (OS.cdf_counts(u, 0.25, eps=0.0) == K // 4).all()
    # uniform rows select the first n blocks (ties to the lower index)
    m = OS.cdf_block_mask(u, 2, 0.125)
    assert m[..., : K // 8].all() and not m[..., K // 8 : K].any() and m[..., K:].all()


def test_layer_selection_cdf_vasc_capacity_is_row_count():
    s = _softmax(np.random.default_rng(12).standard_normal((1, 2, 65, 130)) * 3)
    final, _ = OS.layer_selection(s, mode="topk", sparse_ratio=None, cdf_threshold=0.6, patch_tokens=8288,
                                  total_tokens=8328, official_mask=False)
    n = OS.cdf_counts(s, 0.6)
    last_in = OS.select_top(s, n)[..., 129]
    assert np.array_equal(final[..., :130].sum(-1), n + (~last_in))  # forced mixed tail
    final_v, _ = OS.layer_selection(s, mode="vasc", sparse_ratio=None, cdf_threshold=0.6, patch_tokens=8288,
                                    total_tokens=8328, official_mask=False, state={}, layer_idx=0,
                                    pooled_value=np.random.default_rng(13).standard_normal((1, 2, 130, 64)))
    assert np.array_equal(final_v[..., :130].sum(-1), final[..., :130].sum(-1))
    assert final_v[..., 129].all()


# ---------------------------------------------------------------- PV-execution service
@pytest.mark.parametrize("K", [7, 130, 518])
def test_pv_execution_service_equals_qk_admission_when_every_wave_executes(K):
    """With the PV threshold inert every query warp of a block executes every
    selected child: the exact PV-execution reduction and the QK-admission
    fraction are the same float32 values (the same integers divided)."""
    rng = np.random.default_rng(K)
    Q, W = 9, 4
    sel = rng.random((1, 3, Q, K)) < 0.3
    sel[..., 0] = True
    ex = np.broadcast_to(sel[:, :, :, None, :], (1, 3, Q, W, K)).astype(np.int32)
    assert np.array_equal(OS.pv_execution_service(ex, K).view(np.uint32), OS.qk_service(sel, K).view(np.uint32))


def test_pv_execution_service_counts_skipped_warps():
    """A warp that skips a child lowers that pair's service by 1/(Q*W*pair_size)."""
    Q, W, K = 2, 4, 5  # pairs (0,1), (2,3), (4)
    ex = np.ones((1, 1, Q, W, K), np.int32)
    ex[0, 0, 1, 2, 4] = 0
    ex[0, 0, 0, 0, 1] = 0
    got = OS.pv_execution_service(ex, K)[0, 0]
    assert np.allclose(got, [1 - 1 / (Q * W * 2), 1.0, 1 - 1 / (Q * W)])
