"""GPU parity of the per-head projection kernels (fastAgg.head_proj / head_reduce /
head_wgrad, fast_amd/csrc/head_gemm.hip) with the same products in float64 on the CPU.

The bound is the forward error of a float32 sum of K products: each entry may differ from
the exact value by at most K * 2^-24 * sum_k |a_k b_k| (a loose constant: 4 * K * 2^-24
here), and is checked entry by entry, so a wrong index or a dropped term (an error of the
size of one product) fails for any K below 2^20."""
import pytest
import torch

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _bound_check(got, ref, mag, k, what):
    got = got.double().cpu()
    tol = 4 * k * U * mag + 1e-30
    err = (got - ref).abs()
    bad = err > tol
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} entries out of bound, worst err {float(err.max()):.3e} "
        f"vs tol {float(tol[bad].min()):.3e}")


def _inputs(n, g, j, c, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(n, g * j, generator=gen)
    w = torch.randn(g, j, c, generator=gen)
    y = torch.randn(g, n, c, generator=gen)
    b = torch.randn(g, c, generator=gen)
    return x, w, y, b


SHAPES = [(1000, 2, 50, 376), (77, 8, 32, 708), (33, 1, 5, 13), (16, 3, 64, 100),
          (130, 2, 17, 30), (4099, 1, 100 // 2, 376)]


@pytest.mark.parametrize("shape", SHAPES)
def test_head_proj(dev, shape):
    from fast_amd import fastAgg

    n, g, j, c = shape
    x, w, _, b = _inputs(n, g, j, c, 1, dev)
    xh = x.view(n, g, j).transpose(0, 1).double()           # [g, n, j]
    ref = torch.matmul(xh, w.double()) + b.double()[:, None, :]
    mag = torch.matmul(xh.abs(), w.double().abs()) + b.double().abs()[:, None, :]
    got = fastAgg.head_proj(x.to(dev), w.to(dev), b.to(dev))
    assert got.shape == (g, n, c)
    _bound_check(got, ref, mag, j + 1, "head_proj")
    got0 = fastAgg.head_proj(x.to(dev), w.to(dev), None)
    _bound_check(got0, ref - b.double()[:, None, :], mag, j, "head_proj (no bias)")


@pytest.mark.parametrize("shape", SHAPES)
def test_head_reduce(dev, shape):
    from fast_amd import fastAgg

    n, g, j, c = shape
    _, w, y, _ = _inputs(n, g, j, c, 2, dev)
    ref = torch.matmul(y.double(), w.double().transpose(1, 2).contiguous())   # [g, n, j]
    mag = torch.matmul(y.double().abs(), w.double().abs().transpose(1, 2).contiguous())
    got = fastAgg.head_reduce(y.to(dev), w.to(dev))
    assert got.shape == (n, g * j)
    _bound_check(got.view(n, g, j).transpose(0, 1), ref, mag, c, "head_reduce")
    # a destination-major block read through a permuted view
    yd = y.transpose(0, 1).contiguous().to(dev)                               # [n, g, c]
    got2 = fastAgg.head_reduce(yd.transpose(0, 1), w.to(dev))
    assert torch.equal(got2, got)


# wider heads for the weight gradient (rows_mm's single head of up to D rows): one 128-row
# j group (65 to 128 rows, also with two column workgroups), three and four 64-row j groups
# in one workgroup, more than four (two j workgroups), and column workgroups of those; the
# ones row can open a j group of its own (j = 64, 256)
WGRAD_SHAPES = SHAPES + [(500, 1, 100, 100), (300, 1, 150, 100), (260, 1, 256, 256),
                         (333, 1, 200, 600), (97, 2, 64, 132), (700, 1, 127, 376),
                         (90, 1, 80, 68)]


@pytest.mark.parametrize("shape", WGRAD_SHAPES)
def test_head_wgrad(dev, shape):
    from fast_amd import fastAgg

    n, g, j, c = shape
    x, _, y, _ = _inputs(n, g, j, c, 3, dev)
    xh = x.view(n, g, j).transpose(0, 1).double()                            # [g, n, j]
    ref = torch.matmul(xh.transpose(1, 2).contiguous(), y.double())          # [g, j, c]
    mag = torch.matmul(xh.abs().transpose(1, 2).contiguous(), y.double().abs())
    got = fastAgg.head_wgrad(x.to(dev), y.to(dev), g, True)
    assert got.shape == (g, j + 1, c)
    _bound_check(got[:, :j], ref, mag, n, "head_wgrad")
    _bound_check(got[:, j], y.double().sum(1), y.double().abs().sum(1), n, "head_wgrad ones row")
    again = fastAgg.head_wgrad(x.to(dev), y.to(dev), g, True)
    assert torch.equal(again, got), "head_wgrad is not deterministic"


def test_head_ops_empty(dev):
    from fast_amd import fastAgg

    x = torch.zeros(0, 100, device=dev)
    w = torch.randn(2, 50, 376, device=dev)
    assert fastAgg.head_proj(x, w, None).shape == (2, 0, 376)
    assert fastAgg.head_reduce(torch.zeros(2, 0, 376, device=dev), w).shape == (0, 100)
    dw = fastAgg.head_wgrad(x, torch.zeros(2, 0, 376, device=dev), 2, True)
    assert dw.shape == (2, 51, 376) and not bool(dw.any())


@pytest.mark.parametrize("g,j", [(2, 50), (1, 100)])
def test_head_autograd_matches_float64(dev, g, j):
    """The autograd wrappers of the layer (HeadProj, HeadReduce) against torch autograd in
    float64 on the CPU, through a chain proj -> reduce like the layer's; heads wider than
    the kernels' limit (j = 100) take the batched-GEMM path."""
    from fast_amd.tgat import HeadProj, HeadReduce

    n, c = 500, 376
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(n, g * j, generator=gen)
    wk = torch.randn(g, j, c, generator=gen) * 0.1
    wv = torch.randn(g, j, c, generator=gen) * 0.1
    dz = torch.randn(n, g * j, generator=gen)
    xs = [t.clone().to(dev).requires_grad_(True) for t in (x, wk, wv)]
    z = HeadReduce.apply(torch.tanh(HeadProj.apply(xs[0], xs[1], None)), xs[2])
    z.backward(dz.to(dev))
    rs = [t.clone().double().requires_grad_(True) for t in (x, wk, wv)]
    xh = rs[0].view(n, g, j).transpose(0, 1)
    yh = torch.tanh(torch.matmul(xh, rs[1]))
    zr = torch.matmul(yh, rs[2].transpose(1, 2)).transpose(0, 1).reshape(n, g * j)
    zr.backward(dz.double())
    from tests._util import assert_rel

    assert_rel(z, zr, 1e-5, "chain output")
    for a, b, name in zip(xs, rs, ("dx", "dwk", "dwv")):
        assert_rel(a.grad, b.grad, 1e-5, name)


@pytest.mark.parametrize("n,g,j", [(1000, 2, 50), (77, 8, 32), (5, 1, 100), (300, 3, 7), (0, 2, 50)])
def test_row_group_dots(dev, n, g, j):
    """out[r, h] = a[r, h-block] . b[r, h-block] against float64, entrywise error bound."""
    from fast_amd import fastAgg

    gen = torch.Generator().manual_seed(n + g + j)
    a = torch.randn(n, g * j, generator=gen)
    b = torch.randn(n, g * j, generator=gen)
    got = fastAgg.row_group_dots(a.to(dev), b.to(dev), g)
    assert got.shape == (n, g)
    ref = (a.double().view(n, g, j) * b.double().view(n, g, j)).sum(-1)
    mag = (a.double().abs().view(n, g, j) * b.double().abs().view(n, g, j)).sum(-1)
    _bound_check(got, ref, mag, j, "row_group_dots")


@pytest.mark.parametrize("op", ["proj", "reduce", "wgrad"])
def test_head_ops_wide_magnitudes(dev, op):
    """The split-bf16 kernels (every fp32 operand as three exact bf16 parts) meet the same
    float64 error bound as float32 products when rows and columns span twelve decades
    (scales 10^-6 .. 10^6): the split is exact at every exponent, not only near 1."""
    from fast_amd import fastAgg

    n, g, j, c = 2000, 2, 50, 376
    gen = torch.Generator().manual_seed(11)
    scale = lambda *s: 10.0 ** (torch.rand(*s, generator=gen) * 12 - 6)
    x = torch.randn(n, g * j, generator=gen) * scale(n, 1) * scale(1, g * j)
    w = torch.randn(g, j, c, generator=gen) * scale(g, j, 1) * scale(g, 1, c)
    y = torch.randn(g, n, c, generator=gen) * scale(1, n, 1) * scale(g, 1, c)
    b = torch.randn(g, c, generator=gen) * scale(g, c)
    xh = x.view(n, g, j).transpose(0, 1).double()
    xf = x.view(n, g, j).transpose(0, 1).contiguous()                           # [g, n, j] f32
    if op == "proj":
        got = fastAgg.head_proj(x.to(dev), w.to(dev), b.to(dev))
        f32 = torch.matmul(xf.to(dev), w.to(dev)) + b.to(dev)[:, None, :]
        ref = torch.matmul(xh, w.double()) + b.double()[:, None, :]
        mag = torch.matmul(xh.abs(), w.double().abs()) + b.double().abs()[:, None, :]
        _bound_check(got, ref, mag, j + 1, "head_proj")
    elif op == "reduce":
        got = fastAgg.head_reduce(y.to(dev), w.to(dev)).view(n, g, j).transpose(0, 1)
        f32 = torch.matmul(y.to(dev), w.transpose(1, 2).contiguous().to(dev))
        ref = torch.matmul(y.double(), w.double().transpose(1, 2).contiguous())
        mag = torch.matmul(y.double().abs(), w.double().abs().transpose(1, 2).contiguous())
        _bound_check(got, ref, mag, c, "head_reduce")
    else:
        got = fastAgg.head_wgrad(x.to(dev), y.to(dev), g, True)
        f32 = torch.matmul(xf.transpose(1, 2).contiguous().to(dev), y.to(dev))
        ref = torch.matmul(xh.transpose(1, 2).contiguous(), y.double())
        mag = torch.matmul(xh.abs().transpose(1, 2).contiguous(), y.double().abs())
        _bound_check(got[:, :j], ref, mag, n, "head_wgrad")
        _bound_check(got[:, j], y.double().sum(1), y.double().abs().sum(1), n, "ones row")
        got = got[:, :j]
    # as accurate as a float32 product: the largest error relative to sum |a b| stays within a
    # small factor of torch's float32 GEMM on the same operands (a split into two bf16 parts,
    # or a dropped part product, is 2^8 times worse)
    err = float(((got.double().cpu() - ref).abs() / mag).max())
    err32 = float(((f32.double().cpu() - ref).abs() / mag).max())
    assert err <= 8 * err32 + 1e-12, f"{op}: {err:.3e} against float32 {err32:.3e}"
