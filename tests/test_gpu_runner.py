"""Runner op vasc_residual_norm (include/vasc_runner.h) against torch's bf16 ops.

The residual update must equal torch's bf16 LayerScale multiply and add bit
for bit; the LayerNorm of the updated rows is checked against
torch.nn.functional.layer_norm in float32 of the same bf16 rows (one bf16
rounding apart at most).
"""
import pytest
import torch
import torch.nn.functional as F

from vasc_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("dim,rows", [(512, 7), (1024, 33312 // 16 + 3), (1536, 5), (2048, 130)])
@pytest.mark.parametrize("scaled", [True, False])
def test_residual_norm_matches_torch(dim, rows, scaled):
    g = torch.Generator(device="cuda").manual_seed(dim + rows)
    x = torch.randn(rows, dim, device="cuda", generator=g).to(torch.bfloat16)
    y = (torch.randn(rows, dim, device="cuda", generator=g) * 3).to(torch.bfloat16)
    gamma = (torch.rand(dim, device="cuda", generator=g) * 0.2).to(torch.bfloat16) if scaled else None
    w = (1 + 0.1 * torch.randn(dim, device="cuda", generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(dim, device="cuda", generator=g)).to(torch.bfloat16)
    xn, normed = ops.residual_norm(x, y, gamma, (w, b, 1e-6))
    ref_x = x + (y * gamma if scaled else y)
    assert torch.equal(_bits(xn), _bits(ref_x))
    ref_n = F.layer_norm(ref_x.float(), (dim,), w.float(), b.float(), 1e-6)
    err = (normed.float() - ref_n).abs()
    # bf16 output: within one rounding of the float32 result, element by element
    assert bool((err <= 2 ** -8 * ref_n.abs() + 1e-5).all()), err.max().item()
    # and within one bf16 step of torch's own bf16 LayerNorm
    tb = F.layer_norm(ref_x, (dim,), w, b, 1e-6).float()
    assert bool(((normed.float() - tb).abs() <= 2 ** -7 * tb.abs() + 1e-5).all())
    # residual only: same rows, no norm written
    xo, none = ops.residual_norm(x, y, gamma)
    assert none is None and torch.equal(_bits(xo), _bits(ref_x))


def test_residual_norm_strided_rows_and_defaults():
    """Rows with a stride above dim (a view of a wider tensor); no affine."""
    g = torch.Generator(device="cuda").manual_seed(5)
    wide = torch.randn(9, 3, 1024, device="cuda", generator=g).to(torch.bfloat16)
    x = wide[:, 1]  # row stride 3 * 1024
    y = torch.randn(9, 1024, device="cuda", generator=g).to(torch.bfloat16)
    xn, normed = ops.residual_norm(x, y, None, (None, None, 1e-5))
    ref_x = x + y
    assert torch.equal(_bits(xn), _bits(ref_x))
    ref_n = F.layer_norm(ref_x.float(), (1024,), None, None, 1e-5)
    assert bool(((normed.float() - ref_n).abs() <= 2 ** -8 * ref_n.abs() + 1e-5).all())


def test_residual_norm_argument_errors():
    x = torch.zeros(4, 1000, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(_lib.VascError, match="not built"):
        ops.residual_norm(x, x)
    x = torch.zeros(4, 1024, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.residual_norm(x, x.float())
    with pytest.raises(_lib.VascArgumentError):
        _lib.call("vasc_residual_norm", x.data_ptr(), 1024, x.data_ptr(), 1024, None, None, None, 1e-6, None, 1024,
                  None, 1024, 4, 1024, None)


def test_residual_norm_rejects_fp32_parameters():
    x = torch.zeros(4, 1024, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bf16"):
        ops.residual_norm(x, x, torch.ones(1024, device="cuda"))


def test_block_with_fp32_parameters_takes_the_torch_ops():
    """A bf16 activation stream through a block whose LayerScale and
    LayerNorm parameters are float32 (an fp32 model under autocast): the
    block must not round the parameters to bf16; it matches the same block
    run as torch ops, and a parameter rewritten through ``.data`` is used."""
    from vasc_amd.aggregator import Block
    torch.manual_seed(3)
    blk = Block(512, 8, 2.0).cuda()
    with torch.no_grad():
        blk.ls1.gamma.normal_(0.3, 0.1)
        blk.ls2.gamma.normal_(0.3, 0.1)
        blk.norm2.weight.normal_(1.0, 0.1)
    x = torch.randn(1, 300, 512, device="cuda").to(torch.bfloat16)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = blk(x)
        h = blk.attn(blk.norm1(x))
        ref = x + blk.ls1(h)
        ref = ref + blk.ls2(blk.mlp(blk.norm2(ref)))
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        blk.ls2.gamma.data.copy_(torch.zeros(512))
        out2 = blk(x)
        assert torch.equal(out2.view(torch.int16), (x + blk.ls1(h)).to(out2.dtype).view(torch.int16))
