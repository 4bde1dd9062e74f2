"""Pins the token-layout / norm / rotary oracle (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import layout as OL


def _tokens(N, P, C, B=2):
    # value = 1000 * frame + token-in-frame, so positions are readable
    x = np.zeros((B, N * P, C))
    for n in range(N):
        for t in range(P):
            x[:, n * P + t, :] = 1000 * n + t
    return x


def test_reorder_by_explicit_indices():
    N, P, S = 3, 7, 2
    x = _tokens(N, P, 4)
    r = OL.reorder_to_patch_then_special(x, N, P, S)
    expect = [1000 * n + t for n in range(N) for t in range(S, P)] + [1000 * n + t for n in range(N) for t in range(S)]
    assert r[0, :, 0].tolist() == expect
    assert OL.get_patch_tokens(x, N, P, S)[1, :, 3].tolist() == expect[: N * (P - S)]
    assert OL.get_special_tokens(x, N, P, S)[0, :, 2].tolist() == expect[N * (P - S):]
    assert OL.get_special_tokens(x, N, P, 0) is None


def test_restore_inverts_reorder():
    rng = np.random.default_rng(0)
    for N, P, S in ((2, 5, 1), (4, 9, 5), (3, 6, 0), (1, 3, 3)):
        x = rng.standard_normal((2, 3, N * P, 8))
        assert np.array_equal(OL.restore_to_frame_major(OL.reorder_to_patch_then_special(x, N, P, S), N, P, S), x)


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 64)) * 3 + 1
    w, b = rng.standard_normal(64), rng.standard_normal(64)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), torch.from_numpy(b), 1e-6)
    assert np.allclose(OL.layer_norm(x, w, b, 1e-6), ref.numpy(), rtol=1e-12, atol=1e-12)


def _rope_checks(rope):
    cos, sin = OL.rope_tables(64, 64)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 64))
    zero = np.zeros((4, 2), np.int64)
    assert np.allclose(rope(x, zero, cos, sin), x, atol=0)           # position 0: identity
    pos = np.array([[3, 7], [0, 5], [12, 0], [40, 63]])
    y = rope(x, pos, cos, sin)
    for half in range(2):                                            # each feature pair keeps its norm
        a = x[:, half * 32: half * 32 + 16] ** 2 + x[:, half * 32 + 16: half * 32 + 32] ** 2
        b = y[:, half * 32: half * 32 + 16] ** 2 + y[:, half * 32 + 16: half * 32 + 32] ** 2
        assert np.allclose(a, b, rtol=1e-6)
    # rotations compose: exact float64 tables of p * f
    inv = 1.0 / (100.0 ** (np.arange(0, 32, 2) / 32.0))
    ang = np.arange(128)[:, None] * inv[None]
    c64, s64 = np.cos(ang), np.sin(ang)
    p1, p2 = np.array([[2, 9]] * 4), np.array([[5, 30]] * 4)
    assert np.allclose(rope(rope(x, p1, c64, s64), p2, c64, s64), rope(x, p1 + p2, c64, s64), atol=1e-12)
    # the first feature of each half against the 2x2 rotation written out
    a0 = 3 * inv[0]
    assert np.isclose(y[0, 0], x[0, 0] * np.cos(a0) - x[0, 16] * np.sin(a0), atol=1e-6)
    assert np.isclose(y[0, 16], x[0, 16] * np.cos(a0) + x[0, 0] * np.sin(a0), atol=1e-6)


def test_rope_closed_forms():
    _rope_checks(OL.rope_2d)


def test_rope_checks_catch_a_sign_error():
    def bad(x, pos, cos, sin):  # rotate_half with the sign on the wrong half
        y = OL.rope_2d(x, pos, cos, sin)
        x = np.asarray(x, np.float64)
        p = np.clip(np.asarray(pos)[:, 0], 0, np.asarray(cos).shape[0] - 1)
        c, s = np.asarray(cos, np.float64)[p], np.asarray(sin, np.float64)[p]
        y[..., :16] = x[..., :16] * c + x[..., 16:32] * s
        y[..., 16:32] = x[..., 16:32] * c - x[..., :16] * s
        return y
    with pytest.raises(AssertionError):
        _rope_checks(bad)


def test_pack_layer_order_of_operations():
    # norm before rope before reorder: compare against the steps done by hand
    rng = np.random.default_rng(3)
    N, P, S, H, D = 2, 6, 2, 2, 64
    qkv = rng.standard_normal((1, N * P, 3 * H * D))
    w, b = rng.standard_normal(D), rng.standard_normal(D)
    cos, sin = OL.rope_tables(8, D)
    pos = rng.integers(0, 8, size=(N * P, 2))
    qp, qs, k, v = OL.pack_layer(qkv, N, P, S, H, q_norm=(w, b, 1e-6), k_norm=(None, None, 1e-5), pos=pos,
                                 tables=(cos, sin))
    x = qkv.reshape(1, N * P, 3, H, D)
    q_ref = OL.rope_2d(OL.layer_norm(x[:, :, 0].transpose(0, 2, 1, 3), w, b, 1e-6), pos, cos, sin)
    assert np.allclose(qp, OL.get_patch_tokens(q_ref, N, P, S))
    assert np.allclose(qs, OL.get_special_tokens(q_ref, N, P, S))
    v_ref = x[:, :, 2].transpose(0, 2, 1, 3)
    assert np.array_equal(v, OL.reorder_to_patch_then_special(v_ref, N, P, S))
    assert k.shape == (1, H, N * P, D)


@pytest.mark.parametrize("N,P,S", [(3, 11, 5), (2, 7, 0), (1, 6, 6)])
def test_tokens_helpers_match_oracle(N, P, S):
    """vasc_amd.tokens (the torch drop-in for the reference's
    utils/tokens.py:2-126) against the oracle's index construction."""
    import torch
    from vasc_amd import tokens as T
    x = np.random.default_rng(N * 10 + P).standard_normal((2, 3, N * P, 4)).astype(np.float32)
    xt = torch.from_numpy(x)
    assert np.array_equal(T.get_patch_tokens(xt, N, P, S).numpy(), OL.get_patch_tokens(x, N, P, S))
    sp = T.get_special_tokens(xt, N, P, S)
    ref_sp = OL.get_special_tokens(x, N, P, S)
    assert (sp is None) == (ref_sp is None)
    if sp is not None:
        assert np.array_equal(sp.numpy(), ref_sp)
    re = T.reorder_to_patch_then_special(xt, N, P, S)
    assert np.array_equal(re.numpy(), OL.reorder_to_patch_then_special(x, N, P, S))
    assert np.array_equal(T.restore_to_frame_major(re, N, P, S).numpy(), x)
