"""Installers of the sparse global attention (CPU: module wiring only)."""
import pytest

from vasc_amd import install
from vasc_amd.aggregator import Aggregator, Pi3Decoder


def _small_vggt():
    return Aggregator(dim=128, depth=3, num_heads=2, mlp_ratio=2.0)


def test_vggt_uniform_install_patches_every_global_block():
    agg, store = install.sparse_aggregator_from_vggt(_small_vggt(), sparse_ratio=0.75, verbose=False)
    state = agg._sparse_routing_state
    assert state == {} and store == {0: None, 1: None, 2: None}
    for i, blk in enumerate(agg.global_blocks):
        fwd = blk.attn.forward
        assert fwd.__self__ is blk.attn and blk.attn._sparse_routing_state is state
        assert fwd.__func__.keywords["layer_idx"] == i and fwd.__func__.keywords["sparse_ratio"] == 0.75
    for blk in agg.frame_blocks:
        assert not hasattr(blk.attn, "_sparse_routing_state")


def test_vggt_layerwise_ratios_and_aux_store():
    agg, store = install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.7, 0.8, 0.9],
                                                               aux_output=True, verbose=False)
    assert store == {0: {}, 1: {}, 2: {}}
    assert [b.attn.forward.__func__.keywords["sparse_ratio"] for b in agg.global_blocks] == [0.7, 0.8, 0.9]
    assert agg.global_blocks[1].attn.forward.__func__.keywords["aux_output_store"] is store[1]
    with pytest.raises(ValueError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.5, 0.5], verbose=False)
    with pytest.raises(ValueError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), layer_sparsity_ratios=[0.5, 1.5, 0.5],
                                                      verbose=False)


def test_research_options_are_refused():
    with pytest.raises(NotImplementedError):
        install.sparse_aggregator_from_vggt(_small_vggt(), sparse_ratio=0.75, use_hilbert=True, verbose=False)
    with pytest.raises(NotImplementedError):
        install.sparse_aggregator_from_vggt_layerwise(_small_vggt(), sparse_ratio=0.75, use_radial_layerwise=True,
                                                      verbose=False)
    with pytest.raises(AssertionError):  # neither ratio nor cdf (check_sparse_mode)
        install.sparse_aggregator_from_vggt(_small_vggt(), verbose=False)


def test_pi3_odd_layers_are_global_with_logical_index():
    model = Pi3Decoder(dim=128, depth=6, num_heads=2, mlp_ratio=2.0)
    # the reference checks the uniform mode first (pi3.py:164), so the caller passes sparse_ratio too
    model, store = install.sparse_model_from_pi3(model, sparse_ratio=0.7, layer_sparsity_ratios=[0.6, 0.7, 0.8],
                                                 verbose=False)
    assert sorted(store) == [0, 1, 2]
    for i, blk in enumerate(model.decoder):
        if i % 2:
            kw = blk.attn.forward.__func__.keywords
            assert kw["layer_idx"] == i // 2 and kw["sparse_ratio"] == [0.6, 0.7, 0.8][i // 2]
        else:
            assert not hasattr(blk.attn, "_sparse_routing_state")
    with pytest.raises(ValueError):
        install.sparse_model_from_pi3(Pi3Decoder(dim=128, depth=6, num_heads=2), sparse_ratio=0.5,
                                      layer_sparsity_ratios=[0.5] * 2, verbose=False)


def test_patch_tokens_equal_the_convolution():
    """The runners' patch embedding as one GEMM over non-overlapping patches
    equals the strided convolution (ragged borders dropped as the conv does);
    other convolutions fall back to the module itself."""
    import torch

    from vasc_amd.aggregator import patch_tokens
    torch.manual_seed(0)
    x = torch.randn(3, 3, 70, 85)
    conv = torch.nn.Conv2d(3, 32, 14, 14)
    ref = conv(x).flatten(2).transpose(1, 2)
    got = patch_tokens(conv, x)
    assert got.shape == ref.shape == (3, 30, 32)
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)
    overlap = torch.nn.Conv2d(3, 8, 4, 2)
    assert torch.equal(patch_tokens(overlap, x), overlap(x).flatten(2).transpose(1, 2))


def test_install_for_mode_explicit_arguments():
    """Mode, sparsity and structural allocation as explicit arguments: the
    per-layer ratios of allocation_settings on the backbone's layer-wise
    installer; dense leaves the model unpatched."""
    from vasc_amd import launcher
    agg = Aggregator(dim=128, depth=24, num_heads=2, mlp_ratio=2.0)
    agg, store, settings = install.install_for_mode(agg, "vggt", "vasc", 0.75, verbose=False)
    assert settings["applied"] and settings["layer_sparsities"] == launcher.layer_sparsity("vggt", 0.75, "paper")
    assert [b.attn.forward.__func__.keywords["sparse_ratio"] for b in agg.global_blocks] == settings["layer_sparsities"]
    agg2, store2, s2 = install.install_for_mode(Aggregator(dim=128, depth=24, num_heads=2, mlp_ratio=2.0), "vggt",
                                                "vasc", 0.75, structural_allocation=False, verbose=False)
    assert not s2["applied"] and {b.attn.forward.__func__.keywords["sparse_ratio"] for b in agg2.global_blocks} == {0.75}
    dense = Aggregator(dim=128, depth=24, num_heads=2, mlp_ratio=2.0)
    same, none, sd = install.install_for_mode(dense, "vggt", "dense", 0.75)
    assert same is dense and none is None and sd["effective_policy"] == "dense"
    assert not any(hasattr(b.attn, "_sparse_routing_state") for b in dense.global_blocks)
    pi3, _, sp = install.install_for_mode(Pi3Decoder(dim=128, depth=36, num_heads=2, mlp_ratio=2.0), "pi3", "topk",
                                          0.75, verbose=False)
    glob = [blk for i, blk in enumerate(pi3.decoder) if i % 2]
    assert [b.attn.forward.__func__.keywords["sparse_ratio"] for b in glob] == sp["layer_sparsities"]
    with pytest.raises(ValueError):
        install.install_for_mode(dense, "vggt", "sparse", 0.75)


def test_use_mode_sets_and_restores_the_switches(monkeypatch):
    import os
    from vasc_amd import launcher
    monkeypatch.setenv("SPARSE_VGGT_QK_PV_THRESHOLD", "7")
    monkeypatch.setenv("SPARSE_VGGT_SOMETHING_ELSE", "1")
    with launcher.use_mode("vggt", "vasc") as env:
        now = {k: v for k, v in os.environ.items() if k.startswith("SPARSE_VGGT_")}
        assert now == env == launcher.method_environment("vggt", "vasc")
        assert launcher.routing_config().mode == "vasc" and launcher.routing_config().official_mask
    after = {k: v for k, v in os.environ.items() if k.startswith("SPARSE_VGGT_")}
    assert after == {"SPARSE_VGGT_QK_PV_THRESHOLD": "7", "SPARSE_VGGT_SOMETHING_ELSE": "1"}
