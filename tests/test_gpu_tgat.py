"""GPU parity of the fused TGAT layer (fast_amd.tgat) with the CPU restatement of
layers.py:98-240 (oracle.ref_cpu.tgat_layer) evaluated in float64 on the same float32
inputs: layer output and every gradient within FP32_TOL relative (infinity norm)."""
import numpy as np
import pytest
import torch

from oracle.ref_cpu import layer_params, tgat_layer
from tests._util import FP32_TOL, assert_rel

pytestmark = pytest.mark.gpu


def _mask(E, H, p, seed):
    g = torch.Generator().manual_seed(seed)
    keep = (torch.rand(E, H, generator=g) >= p).float()
    return keep / (1 - p)


def _check_layer(dev, dn, de, dt, H, D, degrees, seed=0, time_bias=False, p_drop=0.0,
                 p_out=0.0, tol=FP32_TOL):
    from fast_amd.tgat import TransfomerAttentionLayer
    from fast_amd.workloads import single_layer

    torch.manual_seed(seed)
    layer = TransfomerAttentionLayer(dn, de, dt, H, 0.0, 0.0, D)
    if time_bias and dt > 0:
        with torch.no_grad():
            layer.time_enc.w.bias.uniform_(-3.0, 3.0)
    layer = layer.to(dev)
    N = len(degrees)
    inp = single_layer(N, dn=dn, de=de, dt_dim=dt, heads=H, dim_out=D, seed=seed + 1,
                       degrees=np.asarray(degrees))
    cpu = inp.block
    blk = cpu.to(dev)
    blk.srcdata["h"].requires_grad_(True)
    E = cpu.num_edges()
    drop = _mask(E, H, p_drop, seed + 2) if p_drop > 0 else None
    out_seed = 1000 + seed
    out = layer.attend(blk, None if drop is None else drop.to(dev), out_drop_seed=out_seed,
                       out_drop_p=p_out)
    out.backward(inp.dout.to(dev))

    P = layer_params(layer)
    h64 = cpu.srcdata["h"].double().requires_grad_(True)
    src, dst = cpu.edges()
    out_drop = None
    if p_out > 0:
        from oracle.ref_cpu import C

        out_drop = torch.from_numpy(C.dropout_mask(N, D, out_seed, p_out))
    ref = tgat_layer(P, h64, cpu.edata["f"], cpu.edata["dt"], src, dst, N, att_drop=drop,
                     out_drop=out_drop)
    ref.backward(inp.dout.double())
    errs = {"out": assert_rel(out, ref, tol, "layer output")}
    for name, prm in layer.named_parameters():
        if P[name].grad is None:
            continue
        errs[name] = assert_rel(prm.grad, P[name].grad, tol, f"grad {name}")
    if dn > 0:
        errs["h"] = assert_rel(blk.srcdata["h"].grad, h64.grad, tol, "grad h")
    return errs


@pytest.mark.parametrize("dims", [(100, 172, 100, 2, 100), (7, 5, 3, 1, 4), (8, 0, 4, 2, 8),
                                  (0, 12, 9, 4, 16), (13, 6, 0, 8, 64), (100, 172, 100, 8, 256),
                                  (200, 172, 100, 1, 64),
                                  # heads of 64 over Kp = 708: W[g] fits neither head_reduce form
                                  # in LDS, so those products fall back to torch GEMMs
                                  (413, 186, 100, 4, 256)])
def test_layer_small(dev, dims):
    dn, de, dt, H, D = dims
    degrees = [0, 1, 2, 3, 10, 10, 17, 0, 20, 5, 64, 70, 1]
    _check_layer(dev, dn, de, dt, H, D, degrees)


def test_layer_wide_head(dev):
    """One head of width 100 (past the per-head kernels' 64: batched GEMMs take the
    projections). The key bias gradient sum_e dscore_e Q[dst(e)] cancels strongly here: a
    plain float32 evaluation of the restatement on the CPU (same inputs, float32 throughout)
    is itself 8.9e-6 from float64, so that one gradient is held to four times the plain
    float32 error; everything else to FP32_TOL."""
    from fast_amd.tgat import TransfomerAttentionLayer
    from fast_amd.workloads import single_layer

    dn, de, dt, H, D = 200, 172, 100, 1, 100
    degrees = [0, 1, 2, 3, 10, 10, 17, 0, 20, 5, 64, 70, 1]
    N = len(degrees)
    torch.manual_seed(0)
    layer = TransfomerAttentionLayer(dn, de, dt, H, 0.0, 0.0, D)
    inp = single_layer(N, dn=dn, de=de, dt_dim=dt, heads=H, dim_out=D, seed=1,
                       degrees=np.asarray(degrees))
    cpu = inp.block
    src, dst = cpu.edges()
    grads = {}
    for dtype in (torch.float64, torch.float32):
        P = layer_params(layer)
        if dtype == torch.float32:
            P = {k: (v.detach().float().requires_grad_(True) if isinstance(v, torch.Tensor) else v)
                 for k, v in P.items()}
        h = cpu.srcdata["h"].detach().to(dtype).clone().requires_grad_(True)
        ref = tgat_layer(P, h, cpu.edata["f"], cpu.edata["dt"], src, dst, N, dtype=dtype)
        ref.backward(inp.dout.to(dtype))
        grads[dtype] = ({k: v.grad for k, v in P.items() if isinstance(v, torch.Tensor)}, h.grad, ref)
    g64, h64, ref64 = grads[torch.float64]
    g32 = grads[torch.float32][0]
    layer = layer.to(dev)
    blk = cpu.to(dev)
    blk.srcdata["h"].requires_grad_(True)
    out = layer.attend(blk)
    out.backward(inp.dout.to(dev))
    assert_rel(out, ref64, FP32_TOL, "layer output")
    assert_rel(blk.srcdata["h"].grad, h64, FP32_TOL, "grad h")
    from tests._util import rel_err

    for name, prm in layer.named_parameters():
        tol = FP32_TOL
        if name == "w_k.bias":
            tol = max(FP32_TOL, 4 * rel_err(g32[name], g64[name]))
        assert_rel(prm.grad, g64[name], tol, f"grad {name}")


def test_layer_time_bias_and_dropout(dev):
    _check_layer(dev, 100, 172, 100, 2, 100, [10] * 50 + [0, 3, 20], time_bias=True, p_drop=0.1,
                 p_out=0.1)


@pytest.mark.parametrize("n,d,p,two,bias", [(1000, 100, 0.0, True, True), (777, 100, 0.3, True, False),
                                            (300, 256, 0.1, False, True), (5, 7, 0.0, True, True),
                                            (0, 100, 0.1, True, True), (4096, 64, 0.2, False, False)])
def test_epilogue_matches_torch(dev, n, d, p, two, bias):
    """LayerNorm(ReLU(dropout(r1 + r2 + bias))) fused kernel vs float64 torch with the same
    hashed multipliers, forward and all gradients."""
    import fast_amd
    from fast_amd.tgat import TgatEpilogue
    from oracle.ref_cpu import C

    g = torch.Generator().manual_seed(n + d)
    r1 = torch.randn(n, d, generator=g)
    r2 = torch.randn(n, d, generator=g) if two else None
    b = torch.randn(d, generator=g) if bias else None
    gamma = 1 + 0.1 * torch.randn(d, generator=g)
    beta = 0.1 * torch.randn(d, generator=g)
    dout = torch.randn(n, d, generator=g)
    seed, eps = 4242, 1e-5
    leaves = [t.to(dev).requires_grad_(True) if t is not None else None
              for t in (r1, r2, b, gamma, beta)]
    out = TgatEpilogue.apply(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], eps, seed, p)
    out.backward(dout.to(dev))
    ref_leaves = [t.double().requires_grad_(True) if t is not None else None
                  for t in (r1, r2, b, gamma, beta)]
    u = ref_leaves[0] + (ref_leaves[1] if two else 0) + (ref_leaves[2] if bias else 0)
    if p > 0:
        u = u * torch.from_numpy(C.dropout_mask(n, d, seed, p)).double()
    ref = torch.nn.functional.layer_norm(torch.relu(u), (d,), ref_leaves[3], ref_leaves[4], eps)
    ref.backward(dout.double())
    if n == 0:
        assert out.shape == (0, d)
        assert torch.count_nonzero(leaves[3].grad) == 0
        if bias:
            assert torch.count_nonzero(leaves[2].grad) == 0
        return
    assert_rel(out, ref, FP32_TOL, "epilogue out")
    for got, want, name in zip(leaves, ref_leaves, ("r1", "r2", "bias", "gamma", "beta")):
        if got is not None:
            assert_rel(got.grad, want.grad, FP32_TOL, f"epilogue grad {name}")
    assert fast_amd.fastAgg is not None


def test_layer_c1_shape(dev):
    """Config 1 shape: 1800 destinations x fanout 10."""
    _check_layer(dev, 100, 172, 100, 2, 100, [10] * 1800, seed=3)


def test_layer_c2_shape(dev):
    """Config 2 shape: 12000 destinations x fanout 10 (forward + backward)."""
    _check_layer(dev, 100, 172, 100, 2, 100, [10] * 12000, seed=4)


def test_layer_ragged(dev):
    from fast_amd.workloads import ragged_degrees

    _check_layer(dev, 100, 172, 100, 2, 100, ragged_degrees(3000, seed=0), seed=5)


def test_gathered_tables_match_dense(dev):
    """Rows gathered inside the kernel from node / edge tables by id give the layer the
    same values as pre-gathered dense features (utils.py:161,187)."""
    from fast_amd.tgat import Block, TransfomerAttentionLayer

    torch.manual_seed(0)
    N, fan, dn, de = 300, 10, 100, 172
    layer = TransfomerAttentionLayer(dn, de, 100, 2, 0.0, 0.0, 100).to(dev)
    g = torch.Generator().manual_seed(9)
    ntab = torch.randn(500, dn, generator=g)
    etab = torch.randn(4000, de, generator=g)
    blk = Block.from_fanout(N, torch.full((N,), fan, dtype=torch.int64))
    E = blk.num_edges()
    nid = torch.randint(0, 500, (N + E,), generator=g)
    eid = torch.randint(0, 4000, (E,), generator=g)
    dt = torch.empty(E).exponential_(1e-4, generator=g)
    a = blk.to(dev)
    a.node_table, a.edge_table = ntab.to(dev), etab.to(dev)
    a.srcdata["ID"], a.edata["ID"], a.edata["dt"] = nid.to(dev), eid.to(dev), dt.to(dev)
    b = blk.to(dev)
    b.srcdata["h"], b.edata["f"], b.edata["dt"] = ntab[nid].to(dev), etab[eid].to(dev), dt.to(dev)
    with torch.no_grad():
        oa, ob = layer(a), layer(b)
    assert torch.equal(oa, ob)


@pytest.mark.parametrize("heads", [1, 2, 4])
def test_missing_rows_read_zero(dev, heads):
    """Row ids outside the tables (negative or past the end) read as zero rows: the layer
    equals the one computed on dense features with those rows zeroed."""
    from fast_amd.tgat import Block, TransfomerAttentionLayer

    torch.manual_seed(1)
    N, dn, de = 200, 100, 172
    layer = TransfomerAttentionLayer(dn, de, 100, heads, 0.0, 0.0, 64).to(dev)
    g = torch.Generator().manual_seed(11)
    ntab = torch.randn(300, dn, generator=g)
    etab = torch.randn(700, de, generator=g)
    deg = torch.randint(0, 40, (N,), generator=g)
    blk = Block.from_fanout(N, deg)
    E = blk.num_edges()
    nid = torch.randint(-50, 350, (N + E,), generator=g)
    eid = torch.randint(-50, 750, (E,), generator=g)
    dt = torch.empty(E).exponential_(1e-4, generator=g)
    a = blk.to(dev)
    a.node_table, a.edge_table = ntab.to(dev), etab.to(dev)
    a.srcdata["ID"], a.edata["ID"], a.edata["dt"] = nid.to(dev), eid.to(dev), dt.to(dev)
    nin, ein = (nid >= 0) & (nid < 300), (eid >= 0) & (eid < 700)
    b = blk.to(dev)
    b.srcdata["h"] = (ntab[nid.clamp(0, 299)] * nin[:, None]).to(dev)
    b.edata["f"] = (etab[eid.clamp(0, 699)] * ein[:, None]).to(dev)
    b.edata["dt"] = dt.to(dev)
    # destination rows (the first N ids) feed the query, outside the fused kernel: keep them
    # in range so that both sides read the same query rows
    a.srcdata["ID"][:N] = nid[:N].clamp(0, 299).to(dev)
    b.srcdata["h"][:N] = ntab[nid[:N].clamp(0, 299)].to(dev)
    with torch.no_grad():
        oa, ob = layer(a), layer(b)
    assert torch.equal(oa, ob)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["exact", "padded", "unaligned"])
def test_table_access_modes(dev, dtype, layout):
    """Rows gathered from float32 / bf16 tables whose rows are chunk-aligned, padded to a
    multiple of 4 or unaligned give exactly the layer computed on the same values given as
    dense float32 features (bf16 widened)."""
    from fast_amd.tgat import Block, TransfomerAttentionLayer

    dn, de = (12, 8) if layout == "exact" else (13, 6)
    ldn, lde = {"exact": (dn, de), "padded": (16, 8), "unaligned": (dn, 7)}[layout]
    torch.manual_seed(0)
    layer = TransfomerAttentionLayer(dn, de, 9, 2, 0.0, 0.0, 16).to(dev)
    g = torch.Generator().manual_seed(5)
    ntab = torch.randn(400, ldn, generator=g).to(dtype)[:, :dn]
    etab = torch.randn(900, lde, generator=g).to(dtype)[:, :de]
    N, fan = 120, 10
    blk = Block.from_fanout(N, torch.full((N,), fan, dtype=torch.int64))
    E = blk.num_edges()
    nid = torch.randint(0, 400, (N + E,), generator=g)
    eid = torch.randint(0, 900, (E,), generator=g)
    dt = torch.empty(E).exponential_(1e-4, generator=g)
    a = blk.to(dev)
    a.node_table, a.edge_table = ntab.to(dev), etab.to(dev)
    a.srcdata["ID"], a.edata["ID"], a.edata["dt"] = nid.to(dev), eid.to(dev), dt.to(dev)
    b = blk.to(dev)
    b.srcdata["h"] = ntab.float()[nid].contiguous().to(dev)
    b.edata["f"] = etab.float()[eid].contiguous().to(dev)
    b.edata["dt"] = dt.to(dev)
    with torch.no_grad():
        oa, ob = layer(a), layer(b)
    assert torch.equal(oa, ob)


def test_two_layer_c5_dims_bf16(dev):
    """Config 5 shapes (node 413, edge 186, time 100, 8 heads, hidden 256) with bf16
    tables (rows padded to 416 / 188) and skewed ids, forward and backward, against the
    float64 restatement evaluated on the same bf16 values."""
    from fast_amd.tgat import TGATEncoder
    from fast_amd.workloads import two_layer

    torch.manual_seed(0)
    enc = TGATEncoder(413, 186, 100, 8, 256, num_layers=2, dropout=0.0, att_dropout=0.0).to(dev)
    inp = two_layer(roots=6, n_nodes=3000, n_edge_rows=20000, dn=413, de=186, heads=8,
                    dim_out=256, seed=2, device="cpu", hot_frac=0.05, hot_share=0.8,
                    dtype=torch.bfloat16, row_align=4)
    blocks = [b.to(dev) for b in inp.blocks]
    out = enc(blocks)
    out.backward(inp.dout.to(dev))

    b0, b1 = inp.blocks
    P0 = layer_params(enc.layers["l0h0"])
    P1 = layer_params(enc.layers["l1h0"])
    h0 = b0.node_table.double()[b0.srcdata["ID"]]
    f0 = b0.edge_table.double()[b0.edata["ID"]]
    s0, d0 = b0.edges()
    r0 = tgat_layer(P0, h0, f0, b0.edata["dt"], s0, d0, b0.num_dst_nodes())
    f1 = b1.edge_table.double()[b1.edata["ID"]]
    s1, d1 = b1.edges()
    r1 = tgat_layer(P1, r0, f1, b1.edata["dt"], s1, d1, b1.num_dst_nodes())
    r1.backward(inp.dout.double())
    assert_rel(out, r1, FP32_TOL, "C5 2-layer output")
    for lname, P in (("l0h0", P0), ("l1h0", P1)):
        for name, prm in enc.layers[lname].named_parameters():
            assert_rel(prm.grad, P[name].grad, FP32_TOL, f"grad {lname}.{name}")


def test_two_layer_stack(dev):
    """2-layer TGAT (modules.py:48-64) on gathered tables vs the float64 restatement."""
    from fast_amd.tgat import TGATEncoder
    from fast_amd.workloads import two_layer

    torch.manual_seed(0)
    enc = TGATEncoder(100, 172, 100, 2, 100, num_layers=2, dropout=0.0, att_dropout=0.0)
    enc = enc.to(dev)
    inp = two_layer(roots=30, n_nodes=2000, n_edge_rows=20000, seed=1, device="cpu")
    blocks = [b.to(dev) for b in inp.blocks]
    out = enc(blocks)
    out.backward(inp.dout.to(dev))

    b0, b1 = inp.blocks
    P0 = layer_params(enc.layers["l0h0"])
    P1 = layer_params(enc.layers["l1h0"])
    h0 = b0.node_table[b0.srcdata["ID"]]
    f0 = b0.edge_table[b0.edata["ID"]]
    s0, d0 = b0.edges()
    r0 = tgat_layer(P0, h0, f0, b0.edata["dt"], s0, d0, b0.num_dst_nodes())
    f1 = b1.edge_table[b1.edata["ID"]]
    s1, d1 = b1.edges()
    r1 = tgat_layer(P1, r0, f1, b1.edata["dt"], s1, d1, b1.num_dst_nodes())
    r1.backward(inp.dout.double())
    assert_rel(out, r1, FP32_TOL, "2-layer output")
    for lname, P in (("l0h0", P0), ("l1h0", P1)):
        for name, prm in enc.layers[lname].named_parameters():
            assert_rel(prm.grad, P[name].grad, FP32_TOL, f"grad {lname}.{name}")


def test_zero_edge_block(dev):
    from fast_amd.tgat import Block, TransfomerAttentionLayer

    layer = TransfomerAttentionLayer(4, 4, 4, 2, 0.0, 0.0, 4).to(dev)
    blk = Block.from_fanout(5, torch.zeros(5, dtype=torch.int64)).to(dev)
    blk.srcdata["h"] = torch.randn(5, 4, device=dev)
    blk.edata["f"] = torch.randn(0, 4, device=dev)
    blk.edata["dt"] = torch.zeros(0, device=dev)
    out = layer(blk)
    assert out.shape == (5, 4) and torch.count_nonzero(out) == 0


def test_dropout_mask_matches_restatement(dev):
    import fast_amd
    from oracle.ref_cpu import C

    for seed, p, E, H in ((0, 0.1, 1000, 2), (2**40 + 12345, 0.5, 777, 8), (7, 0.0, 10, 1)):
        got = fast_amd.fastAgg.dropout_mask(E, H, seed, p, dev).cpu().numpy()
        ref = C.dropout_mask(E, H, seed, p)
        assert (got == ref).all(), (seed, p)
    m = fast_amd.fastAgg.dropout_mask(500_000, 2, 123, 0.1, dev)
    keep = float((m > 0).float().mean())
    assert abs(keep - 0.9) < 0.003, keep


@pytest.mark.parametrize("heads,dim", [(2, 100), (8, 128)])
def test_hashed_dropout_equals_explicit_mask(dev, heads, dim):
    """The kernels' in-kernel dropout (seed, p) gives exactly the layer computed with the
    explicit multipliers fastAgg.dropout_mask(seed, p), forward and backward, and both match
    the restatement with that mask (2 heads: the two-edge kernels; 8: the head-split
    forward and the one-edge backward)."""
    import fast_amd
    from fast_amd.tgat import TransfomerAttentionLayer
    from fast_amd.workloads import single_layer

    torch.manual_seed(0)
    layer = TransfomerAttentionLayer(100, 172, 100, heads, 0.0, 0.3, dim).to(dev)
    degrees = np.array([10] * 100 + [0, 1, 25])
    inp = single_layer(len(degrees), degrees=degrees, seed=3, heads=heads, dim_out=dim)
    seed, p = 99, 0.3
    outs, grads = [], []
    for explicit in (False, True):
        blk = inp.block.to(dev)
        blk.srcdata["h"].requires_grad_(True)
        layer.zero_grad()
        if explicit:
            mask = fast_amd.fastAgg.dropout_mask(blk.num_edges(), heads, seed, p, dev)
            out = layer.attend(blk, drop=mask)
        else:
            out = layer.attend(blk, drop_seed=seed, drop_p=p)
        out.backward(inp.dout.to(dev))
        outs.append(out.detach())
        grads.append([blk.srcdata["h"].grad.clone()] + [q.grad.clone() for q in layer.parameters()])
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(grads[0], grads[1]):
        assert torch.equal(a, b)
    cpu = inp.block
    mask = torch.from_numpy(__import__("oracle.ref_cpu", fromlist=["C"]).C.dropout_mask(
        cpu.num_edges(), heads, seed, p))
    P = layer_params(layer)
    src, dst = cpu.edges()
    ref = tgat_layer(P, cpu.srcdata["h"].double(), cpu.edata["f"], cpu.edata["dt"], src, dst,
                     len(degrees), att_drop=mask)
    assert_rel(outs[0], ref, FP32_TOL, "hashed dropout vs restatement")


@pytest.mark.parametrize("heads", [2, 4])
def test_backward_with_tdot_matches_xbar(dev, heads):
    """The backward given T = dxbar . xbar per destination (tdot) equals the backward that
    reads xbar and forms T itself (both kernel variants: 2 heads take the two-edge kernels)."""
    from fast_amd import fastAgg
    from fast_amd.tgat import kspace_width

    g = torch.Generator().manual_seed(21 + heads)
    N, dn, de, dtd = 300, 100, 172, 100
    deg = torch.randint(0, 30, (N,), generator=g)
    rowptr = torch.zeros(N + 1, dtype=torch.int32)
    rowptr[1:] = torch.cumsum(deg, 0).to(torch.int32)
    E = int(rowptr[-1])
    ntab = torch.randn(500, dn, generator=g)
    etab = torch.randn(900, de, generator=g)
    nid = torch.randint(0, 500, (E,), generator=g)
    eid = torch.randint(0, 900, (E,), generator=g)
    dt = torch.empty(E).exponential_(1e-4, generator=g)
    tw = torch.randn(dtd, generator=g) * 0.1
    tb = torch.randn(dtd, generator=g)
    kp = kspace_width(dn, de, dtd)
    qt = torch.randn(heads, N, kp, generator=g) * 0.05
    dxbar = torch.randn(heads, N, kp, generator=g)
    args = [t.to(dev) for t in (rowptr, ntab, nid, etab, eid, dt, tw, tb, qt)]
    xbar, sc, st = fastAgg.tgat_attn_fwd(*args, 0.2, None)
    dxb = dxbar.to(dev)
    tdot = (dxb * xbar).sum(-1).t().contiguous()       # [N, heads]
    ra = fastAgg.tgat_attn_bwd(*args, 0.2, None, 0, 0.0, xbar, sc, st, dxb, True)
    rb = fastAgg.tgat_attn_bwd(*args, 0.2, None, 0, 0.0, None, sc, st, dxb, True, tdot)
    for x, y, name in zip(ra, rb, ("dqt", "d_node", "d_time_w", "d_time_b")):
        assert_rel(y, x.double(), FP32_TOL, f"tdot backward {name}")


@pytest.mark.parametrize("dims", [(100, 172, 100, 2, 100), (13, 6, 0, 8, 64), (8, 0, 4, 2, 8),
                                  (413, 186, 100, 8, 256)])
def test_layer_params_match_torch(dev, dims):
    """The per-step weight preparation (fastAgg.layer_params_fwd / _bwd through
    tgat.LayerParams) against the same formulas in float64 torch autograd on the CPU:
    K-space weights, the folded query bias product qbk, the w_q / w_out slices, and every
    parameter gradient for random upstream gradients."""
    from fast_amd.tgat import LayerParams, TransfomerAttentionLayer, to_kspace

    dn, de, dt, H, D = dims
    torch.manual_seed(7)
    layer = TransfomerAttentionLayer(dn, de, dt, H, 0.0, 0.0, D)
    with torch.no_grad():
        for p in layer.parameters():
            p.add_(0.1 * torch.randn_like(p))   # non-zero biases everywhere
    names = ["w_q.weight", "w_q.bias", "w_k.weight", "w_k.bias", "w_v.weight", "w_v.bias",
             "time_enc.w.bias", "w_out.weight"]
    pd = dict(layer.named_parameters())
    cpu = [pd[n].detach() if n in pd else None for n in names]
    gpu = [t.to(dev).requires_grad_(True) if t is not None else None for t in cpu]
    ref = [t.double().requires_grad_(True) if t is not None else None for t in cpu]
    outs = LayerParams.apply(*gpu, (H, dn, de, dt))
    wq, bq, wk, bk, wv, bv, bt, wo = ref
    qb = bq + (wq[:, dn:] @ torch.cos(bt) if dt > 0 else 0)
    wk_aug = to_kspace(wk, bk, dn, de, dt)
    kp = wk_aug.shape[1]
    qbk = torch.bmm(qb.view(H, 1, D // H), wk_aug.view(H, D // H, kp)).view(H, kp)
    routs = [wq[:, :dn], wk_aug, to_kspace(wv, bv, dn, de, dt), qbk, wo[:, :D], wo[:, D:]]
    gen = torch.Generator().manual_seed(3)
    ups = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in routs]
    for o, r, name in zip(outs, routs, ["wq_node", "wk_aug", "wv_aug", "qbk", "wo1", "wo2"]):
        assert o.shape == r.shape, name
        assert_rel(o, r, FP32_TOL, f"layer params {name}")
    torch.autograd.backward(list(outs), [u.float().to(dev) for u in ups])
    torch.autograd.backward(routs, ups)
    for g, r, name in zip(gpu, ref, names):
        if g is None:
            continue
        assert_rel(g.grad, r.grad, FP32_TOL, f"layer params grad {name}")


def test_to_blocks_on_device_match_restatement(dev):
    """The pinned, packed transfer to the GPU gives the blocks of the oracle's restatement of
    utils.py:67-87 (sampler results with ragged degrees and zero-degree destinations, more
    results than staging buffers, so buffers are reused after their copy finished), and the
    destination offsets derived on the device equal the restatement's full CSR, whose
    non-empty part is the sampler's cntE (sampler_core.cpp:384-409)."""
    from fast_amd import fastAgg
    from fast_amd.mfg import PinnedStager, to_blocks
    from oracle.ref_cpu import full_rowptr, sampler_cnte, to_dgl_blocks
    from tests.test_host import _assert_block_matches
    from tests.test_oracle import _GoldenSample, _load

    ret = [_GoldenSample(d) for d in _load("mfg.json")["results"]]
    got = to_blocks(ret, hist=1, device=dev, stager=PinnedStager(buffers=2))
    want = to_dgl_blocks(ret, 1)
    assert len(got) == len(want)
    for (b,), (w,), r in zip(got, want, reversed(ret)):
        assert b.device.type == "cuda"
        _assert_block_matches(b, w)
        rp = b.rowptr().cpu().numpy()
        np.testing.assert_array_equal(rp, full_rowptr(r.row(), r.dim_out()))
        # the non-empty destinations' offsets are the sampler's cntE (unique2indptr)
        np.testing.assert_array_equal(np.unique(rp), sampler_cnte(r.row()))
        dst = b.edges()[1]
        if dst.numel():
            ip = fastAgg.exclusive_sum(torch.unique(dst, return_counts=True)[1].to(torch.int32))
            np.testing.assert_array_equal(ip.cpu().numpy(), sampler_cnte(r.row()))
