"""Host-side logic: the launcher mirror and the C-ABI library surface (CPU only)."""
import ctypes
import re
from pathlib import Path

import pytest

from oracle import profile as PR
from vasc_amd import _lib, launcher

ROOT = Path(__file__).resolve().parents[1]


# ------------------------------------------------------------------ launcher
def test_layer_sparsity_matches_oracle_and_string_form():
    for model in ("vggt", "pi3"):
        for s in (0.55, 0.65, 0.75, 0.85, 0.875):
            assert launcher.layer_sparsity(model, s) == PR.layer_sparsity(model, s)
        text = launcher.layer_sparsity_string(model, 0.75, "paper")
        assert all(len(x.split(".")[1]) == 10 for x in text.split(","))


def test_method_environment_release_matrix():
    for model in ("vggt", "pi3"):
        for mode in launcher.MODES:
            env = launcher.method_environment(model, mode)
            assert env["SPARSE_VGGT_QK_PV_THRESHOLD"] == "1e10"
            assert env["SPARSE_VGGT_SKIP_ROUTING_STATS"] == "1"
            assert env["SPARSE_VGGT_COSA_VALUE_RISK_PAIR_DEBT"] == str(int(mode == "vasc"))
            assert ("SPARSE_VGGT_OFFICIAL_MASK" in env) == (model == "vggt" and mode != "dense")
    with pytest.raises(ValueError):
        launcher.method_environment("vggt", "other")


def test_routing_config_resolves_release_modes():
    for model in ("vggt", "pi3"):
        for mode in ("topk", "vasc"):
            cfg = launcher.routing_config(launcher.method_environment(model, mode))
            assert cfg.mode == mode
            assert cfg.official_mask == (model == "vggt")
            assert cfg.skip_routing_stats


def test_routing_config_rejects_research_switches():
    env = launcher.method_environment("vggt", "vasc")
    for extra in ({"SPARSE_VGGT_COSA_ORDERED_LUT": "1"}, {"SPARSE_VGGT_RADIAL_A_DENSE": "1"}):
        with pytest.raises(NotImplementedError):
            launcher.routing_config({**env, **extra})
    for bad in ("-1", "natural_gap:-2", "nan", "abc"):  # as _resolve_qk_pv_threshold (SW:3064-3087)
        with pytest.raises(ValueError):
            launcher.routing_config({**env, "SPARSE_VGGT_QK_PV_THRESHOLD": bad})
    with pytest.raises(ValueError):  # as the reference selector (SW:3999-4000)
        launcher.routing_config({**env, "SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN": "pv_count"})


def test_pv_threshold_resolution():
    import math
    assert launcher.resolve_pv_threshold("sequence_mass_bound", 33312) == math.log(33312.0)
    assert launcher.resolve_pv_threshold("sequence_mass_bound", 1) == math.log(2.0)
    assert launcher.resolve_pv_threshold("natural_gap:2", 10) == 2 * math.log2(math.e)
    assert launcher.resolve_pv_threshold("1e10", 10) == 1e10
    assert launcher.pv_threshold_active("", 5) and launcher.pv_threshold_active(" 0, 7,15 ", 7)
    assert not launcher.pv_threshold_active("0,7,15", 8)
    env = {**launcher.method_environment("pi3", "vasc"), "SPARSE_VGGT_QK_PV_THRESHOLD": "sequence_mass_bound",
           "SPARSE_VGGT_QK_PV_ACTIVE_LAYERS": "1,3"}
    cfg = launcher.routing_config(env)
    assert cfg.pv_threshold == "sequence_mass_bound" and cfg.pv_active_layers == "1,3"


def test_routing_config_service_domains():
    env = launcher.method_environment("pi3", "vasc")
    assert launcher.routing_config(env).service_domain == "qk_admission"
    cfg = launcher.routing_config({**env, "SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN": "pv_execution"})
    assert cfg.mode == "vasc" and cfg.service_domain == "pv_execution"
    env.pop("SPARSE_VGGT_COSA_DEBT_SERVICE_DOMAIN")  # the reference's default domain
    assert launcher.routing_config(env).service_domain == "pv_execution"


def test_allocation_settings():
    a = launcher.allocation_settings("vggt", "vasc", 0.75, True)
    assert a["applied"] and a["effective_policy"] == "paper" and len(a["layer_sparsities"]) == 24
    d = launcher.allocation_settings("vggt", "dense", 0.75, True)
    assert not d["applied"] and d["layer_sparsities"] == [0.0] * 24
    u = launcher.allocation_settings("pi3", "topk", 0.65, True)
    assert u["effective_policy"] == "uniform" and u["layer_sparsities"] == [0.65] * 18


# ------------------------------------------------------------------ C-ABI
def _header_functions():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(vasc_\w+)\s*\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert names == set(_lib.SIGNATURES), "ctypes table out of sync with include/*.h"
    assert lib.vasc_abi_version() == 5


def test_host_only_queries_and_argument_errors():
    lib = _lib.load()
    # per row: total, row pair sum, capacity (fp32/int32); per pair: admitted
    # debt, (innovation, debt) pair, service counts; per 32-row chunk and
    # pair: a float64 partial of the arrival mean; per head: 3 gate partials;
    # per row: the select pass's fast-path flag.
    def al(x):
        return (x + 255) // 256 * 256
    BH, Q, K = 16, 259, 518
    P, chunks = (K + 1) // 2, -(-Q // 32)
    expect = 3 * al(BH * Q * 4) + al(BH * P * 4) + al(BH * P * 8) + al(BH * chunks * P * 8) + al(BH * 3 * 8) \
        + al(BH * P * 4) + al(BH * Q * 4)
    assert lib.vasc_select_workspace_size(1, BH, Q, K) == expect
    assert lib.vasc_select_workspace_size(0, 16, 259, 518) == 0
    # result regions: row totals, row pair sums, capacities, then the admitted debt
    offs = [lib.vasc_select_workspace_offset(1, BH, Q, K, r) for r in range(4)]
    assert offs == [0, al(BH * Q * 4), 2 * al(BH * Q * 4), 3 * al(BH * Q * 4)]
    assert lib.vasc_select_workspace_offset(1, BH, Q, K, 7) == -1
    assert lib.vasc_select_workspace_offset(0, BH, Q, K, 0) == -1
    assert lib.vasc_packed_v_elems(1, 16, 33312, 64) == 16 * 521 * 64 * 64
    # validation happens before any HIP call: these return without a GPU
    rc = lib.vasc_pack_v(None, 0, 0, 8, 1, 1, 64, 64, None, None)
    assert rc == 1 and b"required" in lib.vasc_last_error()
    rc = lib.vasc_pack_v(None, 0, 0, 8, 1, 1, 64, 128, None, None)
    assert rc == 2 and b"head_dim" in lib.vasc_last_error()
    rc = lib.vasc_block_sparse_attn_fwd(None, 0, 0, 8, None, 0, 0, 8, None, None, 0, 0, 8, 1, 1, 128, 64, 64,
                                        None, 1, None, 0, ctypes.c_float(0.125), None)
    assert rc == 1
    with pytest.raises(_lib.VascArgumentError):
        _lib.call("vasc_settle_terminal", None, None, None, 0, None, None)
    # token layout: sizes and pointers are checked before any launch
    f = ctypes.c_float
    rc = lib.vasc_pack_qkv(None, 0, 3072, 64, None, 0, 3072, 64, None, 0, 3072, 64, 1, 16, 2, 1041, 5, 64,
                           None, None, f(1e-6), 0, None, None, f(1e-6), 0, None, 0, 2, None, None, 0,
                           None, None, None, None, None)
    assert rc == 1 and b"q is NULL" in lib.vasc_last_error()
    rc = lib.vasc_pack_qkv(None, 0, 3072, 64, None, 0, 3072, 64, None, 0, 3072, 64, 1, 16, 2, 1041, 5, 128,
                           None, None, f(1e-6), 0, None, None, f(1e-6), 0, None, 0, 2, None, None, 0,
                           None, None, None, None, None)
    assert rc == 2 and b"head_dim" in lib.vasc_last_error()
    # v may be absent when v_out is (q and k only); k_out may not
    fake = ctypes.c_void_p(256)  # aligned, never dereferenced: validation stops first
    rc = lib.vasc_pack_qkv(fake, 0, 3072, 64, fake, 0, 3072, 64, None, 0, 0, 0, 1, 16, 2, 1041, 5, 64,
                           None, None, f(1e-6), 0, None, None, f(1e-6), 0, None, 0, 2, None, None, 0,
                           fake, fake, None, None, None)
    assert rc == 1 and b"k_out is required" in lib.vasc_last_error()
    rc = lib.vasc_pack_qkv(fake, 0, 3072, 64, fake, 0, 3072, 64, None, 0, 0, 0, 1, 16, 2, 1041, 5, 64,
                           None, None, f(1e-6), 0, None, None, f(1e-6), 0, None, 0, 2, None, None, 0,
                           None, fake, fake, None, None)
    assert rc == 1 and b"q_patch is required" in lib.vasc_last_error()
    rc = lib.vasc_pack_qkv(fake, 0, 3072, 64, fake, 0, 3072, 64, None, 0, 3072, 64, 1, 16, 2, 1041, 5, 64,
                           None, None, f(1e-6), 0, None, None, f(1e-6), 0, None, 0, 2, None, None, 0,
                           fake, fake, fake, fake, None)
    assert rc == 1 and b"v is NULL" in lib.vasc_last_error()
    rc = lib.vasc_restore_tokens(None, 0, 0, 8, None, 0, 0, 8, 1, 16, 2, 1041, 5, 64, None, None)
    assert rc == 1 and b"out must be" in lib.vasc_last_error()
    rc = lib.vasc_restore_tokens(None, 0, 0, 8, None, 0, 0, 8, 1, 16, 2, 4, 5, 64, None, None)
    assert rc == 1 and b"invalid sizes" in lib.vasc_last_error()
    rc = lib.vasc_global_attn_fwd(None, 0, 0, 8, None, 0, 0, 8, None, 0, 0, 8, None, None, 0, 0, 8,
                                  None, 0, 0, 8, 1, 1, 128, 32, 64, 64, None, 1, None, f(0.125), None)
    assert rc == 1 and b"q_special" in lib.vasc_last_error()
    # cdf counts: pointers, the built key-block range and the ratio floor (never dereferenced here)
    fake = ctypes.c_void_p(256)
    rc = lib.vasc_cdf_counts(None, 1, 16, 259, 518, fake, 0, 0, fake, None, None)
    assert rc == 1 and b"required" in lib.vasc_last_error()
    rc = lib.vasc_cdf_counts(fake, 1, 16, 259, 9000, fake, 0, 0, fake, None, None)
    assert rc == 2 and b"8192" in lib.vasc_last_error()
    rc = lib.vasc_cdf_counts(fake, 1, 16, 259, 518, fake, 519, 0, fake, None, None)
    assert rc == 1 and b"min_count" in lib.vasc_last_error()
    rc = lib.vasc_block_sparse_attn_pv_fwd(None, 0, 0, 8, None, 0, 0, 8, None, None, 0, 0, 8, 1, 1, 128, 64, 64,
                                           None, 1, None, 0, ctypes.c_float(0.125), None, None, None)
    assert rc == 1 and b"pv_threshold" in lib.vasc_last_error()
    # token-major global attention: frame sizes and the key count are checked first
    rc = lib.vasc_global_attn_tokens_fwd(fake, 0, 0, 8, fake, 0, 0, 8, fake, 0, 0, 8, fake, fake, 1, 1, 2, 5, 5,
                                         10, 64, fake, 1, fake, f(0.125), None)
    assert rc == 1 and b"frame sizes" in lib.vasc_last_error()
    rc = lib.vasc_global_attn_tokens_fwd(fake, 0, 0, 8, fake, 0, 0, 8, fake, 0, 0, 8, fake, fake, 1, 1, 2, 6, 1,
                                         10, 64, fake, 1, fake, f(0.125), None)
    assert rc == 1 and b"N*P" in lib.vasc_last_error()
    # runner op: built widths, required rows, outputs and alignment
    rc = lib.vasc_residual_norm(fake, 1000, fake, 1000, None, None, None, f(1e-6), fake, 1000, None, 0, 4, 1000, None)
    assert rc == 2 and b"not built" in lib.vasc_last_error()
    rc = lib.vasc_residual_norm(fake, 1024, None, 1024, None, None, None, f(1e-6), fake, 1024, None, 0, 4, 1024, None)
    assert rc == 1 and b"y is NULL" in lib.vasc_last_error()
    rc = lib.vasc_residual_norm(fake, 1024, fake, 1024, None, None, None, f(1e-6), None, 0, None, 0, 4, 1024, None)
    assert rc == 1 and b"both NULL" in lib.vasc_last_error()
    rc = lib.vasc_residual_norm(fake, 1000, fake, 1024, None, None, None, f(1e-6), fake, 1024, None, 0, 4, 1024, None)
    assert rc == 1 and b"row stride" in lib.vasc_last_error()


def test_select_rejects_ledger_aliasing():
    """The ledger cannot be updated in place: the VASC head pass reads all of a
    head's ledger inputs while other workgroups write its outputs. Overlapping
    output/input ranges are rejected before any launch."""
    lib = _lib.load()
    B, H, Q, K = 1, 2, 3, 10
    P = (K + 1) // 2
    n = B * H * P * 4  # bytes of one ledger tensor
    base = 1 << 20
    fake = lambda off: ctypes.c_void_p(base + off)  # noqa: E731 (never dereferenced)
    score, inn, idx, cnt, ws = fake(0), fake(4096), fake(8192), fake(12288), fake(16384)
    d_in, pend, prev = fake(65536), fake(65536 + 4096), fake(65536 + 8192)

    def call(debt_out, arrival_out, service_out):
        return lib.vasc_select_blocks(score, inn, B, H, Q, K, _lib.MODE_VASC, 3, None, None, 0, 3, 0,
                                      d_in, pend, prev, debt_out, arrival_out, service_out, None, None, None,
                                      idx, 3, cnt, ws, 1 << 20, None)

    for outs in ((d_in, fake(20480), fake(24576)),           # debt updated in place
                 (fake(20480), pend, fake(24576)),           # arrival over pending
                 (fake(20480), fake(24576), prev),           # service over prev_service
                 (fake(65536 + 4), fake(20480), fake(24576)),  # partial overlap
                 (fake(20480), fake(20480 + n - 4), fake(24576))):  # outputs overlapping each other
        assert call(*outs) == 1
        assert b"overlap" in lib.vasc_last_error()

