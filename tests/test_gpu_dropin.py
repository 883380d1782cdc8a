"""GPU parity of the drop-in fastAgg operators against the CPU restatement (oracle/).

Integer bookkeeping is compared bit-exactly; float results within FP32_TOL relative
(infinity-norm over the tensor)."""
import numpy as np
import pytest
import torch

from oracle.ref_cpu import C
from tests._util import FP32_TOL, assert_equal, assert_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fa():
    import fast_amd

    return fast_amd.fastAgg


def _csr(degrees, rng=None):
    deg = np.asarray(degrees, dtype=np.int64)
    nz = deg[deg > 0]
    indptr = np.concatenate([[0], np.cumsum(nz)]).astype(np.int32)
    dst = np.repeat(np.arange(deg.size), deg).astype(np.int64)
    return indptr, dst


DEGREE_SETS = {
    "fanout10": [10] * 300,
    "ragged": [0, 1, 2, 3, 5, 0, 17, 20, 64, 65, 100, 1, 0, 7],
    "single": [1],
}


# ---------------------------------------------------------------------------------------
# bookkeeping (bit-exact)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [0, 1, 7, 2047, 2048, 2049, 100_003, 1_000_000])
def test_exclusive_sum(fa, dev, n):
    rng = np.random.default_rng(n)
    x = rng.integers(0, 50, size=n).astype(np.int32)
    got = fa.exclusive_sum(torch.from_numpy(x).to(dev))
    assert_equal(got, C.exclusive_sum(x), "exclusive_sum")


def test_exclusive_sum_wraps(fa, dev):
    x = np.full(5000, 2**30, dtype=np.int32)
    got = fa.exclusive_sum(torch.from_numpy(x).to(dev))
    assert_equal(got, C.exclusive_sum(x), "exclusive_sum wrap")


@pytest.mark.parametrize("layout", ["random", "sorted", "runs"])
@pytest.mark.parametrize("n_ids,n_nodes", [(0, 5), (1000, 17), (300_000, 1000), (5000, 1),
                                           (1_192_133, 200_000)])
def test_cal_deg(fa, dev, n_ids, n_nodes, layout):
    """Bit-exact degrees; sorted ids and runs of repeated ids (counted once per run within a
    wave, runs crossing wave boundaries, out-of-range ids inside runs) as the sampler lays
    them out, and random ids."""
    rng = np.random.default_rng(n_ids)
    ids = rng.integers(-3, n_nodes + 3, size=n_ids).astype(np.int32)
    if layout == "sorted":
        ids = np.sort(ids)
    elif layout == "runs":
        ids = np.repeat(ids, rng.integers(1, 90, size=n_ids))[:n_ids]
    got = fa.cal_deg(torch.from_numpy(ids).to(dev), n_nodes)
    assert_equal(got, C.cal_deg(ids, n_nodes), "cal_deg")


@pytest.mark.parametrize("n,threshold", [(1, 3), (2, 1), (300, 7), (1025, 16), (70_001, 5),
                                         (513, -4)])
def test_get_balanced_ptr(fa, dev, n, threshold):
    rng = np.random.default_rng(n)
    ptr = np.concatenate([[0], np.cumsum(rng.integers(0, 20, size=n - 1))]).astype(np.int32)
    got = fa.getBalancedPtr(torch.from_numpy(ptr).to(dev), threshold)
    assert_equal(got, C.balance_mask(ptr, threshold), "getBalancedPtr")


def test_get_balanced_ptr_nonmonotone(fa, dev):
    rng = np.random.default_rng(5)
    ptr = rng.integers(-100, 100, size=600).astype(np.int32)
    got = fa.getBalancedPtr(torch.from_numpy(ptr).to(dev), 9)
    assert_equal(got, C.balance_mask(ptr, 9), "getBalancedPtr non-monotone")


@pytest.mark.parametrize("name", list(DEGREE_SETS))
def test_rowptr_from_dst(fa, dev, name):
    deg = DEGREE_SETS[name]
    _, dst = _csr(deg)
    got = fa.rowptr_from_dst(torch.from_numpy(dst).to(dev), len(deg))
    assert_equal(got, C.rowptr(dst, len(deg)), "rowptr")


def test_unique2indptr_matches_cnte(fa, dev):
    from fast_amd.efficientGOP import unique2indptr

    deg = DEGREE_SETS["ragged"]
    indptr, dst = _csr(deg)
    got = unique2indptr(torch.from_numpy(dst).to(dev), len(deg))
    assert_equal(got, indptr, "unique2indptr")


# ---------------------------------------------------------------------------------------
# segmented softmax
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", list(DEGREE_SETS))
@pytest.mark.parametrize("heads", [1, 2, 8])
def test_edge_softmax_fwd_bwd(fa, dev, name, heads):
    indptr, dst = _csr(DEGREE_SETS[name])
    E = dst.size
    rng = np.random.default_rng(heads)
    x = (rng.standard_normal((E, heads)) * 3).astype(np.float32)
    dy = rng.standard_normal((E, heads)).astype(np.float32)
    ti, tx = torch.from_numpy(indptr).to(dev), torch.from_numpy(x).to(dev)
    y = fa.forward_edge_softmax(ti, ti, tx, 512, heads)[0]
    y_ref = C.edge_softmax_fwd(indptr, x, heads, 0)
    assert_rel(y, y_ref, 1e-6, "forward_edge_softmax")
    dx = fa.backward_edge_softmax(ti, ti, torch.from_numpy(dy).to(dev), y, 512, heads)[0]
    assert_rel(dx, C.edge_softmax_bwd(indptr, dy, y.cpu().numpy(), heads), 1e-6,
               "backward_edge_softmax")
    yc = fa.forward_csr_edge_softmax(ti, ti, tx, 32, 16)[0]
    assert_rel(yc, C.edge_softmax_fwd(indptr, x, heads, 1), 1e-6, "forward_csr_edge_softmax")
    dxc = fa.backward_csr_edge_softmax(ti, ti, torch.from_numpy(dy).to(dev), yc, 32, 16)[0]
    assert_rel(dxc, C.edge_softmax_bwd(indptr, dy, yc.cpu().numpy(), heads), 1e-6,
               "backward_csr_edge_softmax")


@pytest.mark.parametrize("layout", ["tiles", "wide", "mixed"])
@pytest.mark.parametrize("heads", [1, 2, 8])
def test_edge_softmax_many_segments(fa, dev, layout, heads):
    """Many segments per launch: empty segments among short ones, edges before the first
    offset and after the last (zeros), runs of long segments (40 and 70 edges) and both
    kinds in one launch; forward (both forms) and backward."""
    rng = np.random.default_rng(heads + len(layout))
    if layout == "tiles":
        deg = rng.integers(0, 21, size=1000)
    elif layout == "wide":
        deg = np.full(600, 40)
    else:   # tiles of short and of long segments in turn
        deg = np.concatenate([rng.integers(0, 8, size=256), np.full(256, 70),
                              rng.integers(0, 8, size=300)])
    indptr = np.concatenate([[7], 7 + np.cumsum(deg)]).astype(np.int32)
    E = int(indptr[-1]) + 5
    x = (rng.standard_normal((E, heads)) * 3).astype(np.float32)
    dy = rng.standard_normal((E, heads)).astype(np.float32)
    ti, tx = torch.from_numpy(indptr).to(dev), torch.from_numpy(x).to(dev)
    for mode, fwd in ((0, fa.forward_edge_softmax), (1, fa.forward_csr_edge_softmax)):
        y = fwd(ti, ti, tx, 512, heads)[0] if mode == 0 else fwd(ti, ti, tx, 32, 16)[0]
        assert_rel(y, C.edge_softmax_fwd(indptr, x, heads, mode), 1e-6, f"forward mode {mode}")
        assert not y[:7].any() and not y[-5:].any()
    dx = fa.backward_edge_softmax(ti, ti, torch.from_numpy(dy).to(dev), y, 512, heads)[0]
    assert_rel(dx, C.edge_softmax_bwd(indptr, dy, y.cpu().numpy(), heads), 1e-6, "backward")
    assert not dx[:7].any() and not dx[-5:].any()


def test_edge_softmax_partial_heads(fa, dev):
    """num_heads below the input width: only the first num_heads columns (edge_softmax.cu:66)."""
    indptr, dst = _csr([3, 4, 0, 2])
    x = np.random.default_rng(0).standard_normal((dst.size, 4)).astype(np.float32)
    ti = torch.from_numpy(indptr).to(dev)
    y = fa.forward_edge_softmax(ti, ti, torch.from_numpy(x).to(dev), 512, 2)[0]
    assert tuple(y.shape) == (dst.size, 2)
    assert_rel(y, C.edge_softmax_fwd(indptr, x, 2, 0), 1e-6, "partial heads")


def test_edge_softmax_f64(fa, dev):
    indptr, dst = _csr(DEGREE_SETS["ragged"])
    x = torch.randn(dst.size, 2, dtype=torch.float64)
    y = fa.forward_edge_softmax(torch.from_numpy(indptr).to(dev), torch.from_numpy(indptr).to(dev),
                                x.to(dev), 512, 2)[0].cpu()
    ref = torch.zeros_like(x)
    for s in range(indptr.size - 1):
        lb, le = indptr[s], indptr[s + 1]
        ref[lb:le] = torch.softmax(x[lb:le], 0)
    assert_rel(y, ref, 1e-13, "f64 softmax")


def test_balanced_softmax(fa, dev):
    rng = np.random.default_rng(3)
    B, maxn, H = 40, 16, 2
    counts = rng.integers(0, maxn + 1, size=B)
    bptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    E = int(bptr[-1])
    key = rng.integers(0, 5, size=(B, maxn)).astype(np.int64)
    key[0, 0] = -1   # skipped entry
    x = rng.standard_normal((E, H)).astype(np.float32)
    dy = rng.standard_normal((E, H)).astype(np.float32)
    tb, tk = torch.from_numpy(bptr).to(dev), torch.from_numpy(key).to(dev)
    y = fa.forward_balanced_edge_softmax(tb, tk, torch.from_numpy(x).to(dev), 64, 16)[0]
    y_ref = C.group_softmax_fwd(bptr, key, x)
    assert_rel(y, y_ref, 1e-6, "forward_balanced_edge_softmax")
    dx = fa.backward_balanced_edge_softmax(tb, tk, torch.from_numpy(dy).to(dev), y, 64, 16)[0]
    assert_rel(dx, C.group_softmax_bwd(bptr, key, dy, y.cpu().numpy()), 1e-6,
               "backward_balanced_edge_softmax")


# ---------------------------------------------------------------------------------------
# aggregation
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", list(DEGREE_SETS))
@pytest.mark.parametrize("dim", [1, 100, 300])
def test_tgat_aggregation(fa, dev, name, dim):
    deg = DEGREE_SETS[name]
    indptr, dst = _csr(deg)
    N, E = len(deg), dst.size
    src = np.arange(N, N + E, dtype=np.int64)
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((N + E, dim)).astype(np.float32)
    dout = rng.standard_normal((N, dim)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    # forward_tgat: out[dst] += x[src]; the reference passes (edges()[1], edges()[0], ...).
    out = fa.forward_tgat(t(dst), t(src), t(x), N, 8, 128)[0]
    ref = C.edge_scatter_sum(dst, src, x, N)
    assert_rel(out, ref, FP32_TOL, "forward_tgat")
    out_s = fa.forward_tgat_shd(t(indptr), t(indptr), t(dst), t(src), t(x), N, 8, 32)[0]
    assert_rel(out_s, C.segment_sum(indptr, dst, src, x, N), FP32_TOL, "forward_tgat_shd")
    # backward: d_x[src] += d_out[dst]
    dx = fa.backward_tgat(t(dst), t(src), t(dout), N + E, 8, 128)[0]
    assert_rel(dx, C.edge_scatter_sum(src, dst, dout, N + E), FP32_TOL, "backward_tgat")
    dxs = fa.backward_tgat_shd(t(indptr), t(indptr), t(dst), t(src), t(dout), N + E, 8, 32)[0]
    assert_rel(dxs, C.edge_scatter_sum(src, dst, dout, N + E, indptr), FP32_TOL,
               "backward_tgat_shd")
    # empty destinations stay exactly zero
    empty = np.asarray(deg) == 0
    assert torch.count_nonzero(out[torch.from_numpy(empty).to(dev)]) == 0


@pytest.mark.parametrize("dim", [7, 100, 300, 600])
def test_segment_sum_edge_cases(fa, dev, dim):
    """forward_tgat_shd over segments taken two at a time by half-waves: empty segments,
    destinations below 0 and past n_out (skipped), segments of 1 to 100 edges side by side
    (the halves step to the longer one's end), an odd segment count, offsets past the edge
    count (clamped), missing source rows; rows no segment writes stay zero."""
    rng = np.random.default_rng(dim)
    lens = [3, 0, 1, 100, 33, 0, 32, 64, 2, 65, 7, 0, 5]
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    E = int(indptr[-1])
    indptr = np.concatenate([indptr, [E + 5]]).astype(np.int32)   # a segment past the edges
    n_out = 20
    seg_dst = np.array([0, 1, -2, 3, 4, 5, 25, 7, 8, 9, 10, 11, 19, 12])
    dst = np.repeat(seg_dst[:len(lens)], lens).astype(np.int64)
    src = rng.integers(-2, 260, size=E).astype(np.int64)           # some rows missing
    x = rng.standard_normal((250, dim)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    out = fa.forward_tgat_shd(t(indptr), t(indptr), t(dst), t(src), t(x), n_out, 8, 32)[0]
    assert_rel(out, C.segment_sum(indptr, dst, src, x, n_out), FP32_TOL, "forward_tgat_shd")


def test_tgat_aggregation_unsorted(fa, dev):
    rng = np.random.default_rng(11)
    E, N, S = 5000, 300, 900
    dst = rng.integers(0, N, size=E).astype(np.int64)
    src = rng.integers(0, S, size=E).astype(np.int64)
    x = rng.standard_normal((S, 64)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    out = fa.forward_tgat(t(dst), t(src), t(x), N, 8, 128)[0]
    assert_rel(out, C.edge_scatter_sum(dst, src, x, N), FP32_TOL, "unsorted forward_tgat")


@pytest.mark.parametrize("case", ["gaps", "out_of_range", "one_long_run", "tile_sorted_only",
                                  "no_edges", "csr_subrange", "distinct", "distinct_gap",
                                  "pair_at_tile_edge", "distinct_out_of_range"])
@pytest.mark.parametrize("dim", [7, 100, 600])
def test_tgat_aggregation_sorted_edge_cases(fa, dev, case, dim):
    """The run-owner path of the scatter (sorted output index, plain stores, every output row
    written) and its switch to the atomic path: rows before, between and after the runs come
    out zero, indices outside [0, n_out) are skipped, a run spanning many 64-edge tiles is one
    sum, an index sorted inside every tile but not across tiles takes the atomic path; against
    the C restatement (which starts from zeros). The "distinct" cases cover the tiles whose
    every edge is a run of its own (copied row by row): with no gap, with a gap inside a tile,
    with the last run of a tile going on into the next tile, and with indices below 0 and
    past n_out."""
    rng = np.random.default_rng(dim + len(case))
    n_out, indptr = 40, None
    if case == "gaps":
        dst = np.repeat([3, 4, 9, 30], [2, 70, 1, 5])
    elif case == "out_of_range":
        dst = np.array([-3, -3, -1, 0, 0, 5, 5, 5, 39, 40, 40, 41, 100])
    elif case == "one_long_run":
        dst = np.full(1000, 17)
    elif case == "tile_sorted_only":
        dst = np.concatenate([np.repeat([20, 21], 32), np.repeat([2, 3], 32), np.full(64, 20)])
    elif case == "no_edges":
        dst = np.zeros(0)
    elif case == "distinct":
        dst, n_out = np.arange(3, 133), 140
    elif case == "distinct_gap":
        dst, n_out = np.concatenate([np.arange(0, 50), np.arange(52, 120)]), 130
    elif case == "pair_at_tile_edge":
        dst, n_out = np.concatenate([np.arange(0, 64), [63], np.arange(64, 100)]), 100
    elif case == "distinct_out_of_range":
        dst = np.arange(-3, 140)
    else:
        dst = np.repeat(np.arange(0, 40, 3), 7)
        indptr = np.array([5, 20, 20, 61], dtype=np.int32)   # edges 5..60 only
    dst = dst.astype(np.int64)
    E = dst.size
    src = rng.integers(0, 300, size=E).astype(np.int64)
    x = rng.standard_normal((300, dim)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    ref = C.edge_scatter_sum(dst, src, x, n_out, indptr)
    if indptr is None:
        out = fa.forward_tgat(t(dst), t(src), t(x), n_out, 8, 128)[0]
        what = f"forward_tgat {case}"
    else:
        # backward_tgat_shd(indptr, indices, dst_edges, src_edges, d_input, src_nodes, ...)
        # scatters d_input[dst_edges[e]] into rows src_edges[e] over the CSR-covered edges
        out = fa.backward_tgat_shd(t(indptr), t(indptr), t(src), t(dst), t(x), n_out, 8, 32)[0]
        what = f"backward_tgat_shd {case}"
    assert_rel(out, ref, FP32_TOL, what)
    hit = np.zeros(n_out, bool)
    lo, hi = (0, E) if indptr is None else (int(indptr[0]), int(indptr[-1]))
    hit[[d for d in dst[lo:hi] if 0 <= d < n_out]] = True
    assert torch.count_nonzero(out[torch.from_numpy(~hit).to(dev)]) == 0, "rows without edges"


def test_edge_softmax_rows_outside_segments_are_zero(fa, dev):
    """Edges before the first segment and after the last one get zeros (the outputs are not
    zero-filled beforehand); both the row kernels (2 heads) and the per-thread kernel
    (3 heads) are covered, forward and backward."""
    indptr = np.array([3, 5, 5, 9], dtype=np.int32)
    for heads in (2, 3):
        x = np.random.default_rng(heads).standard_normal((12, heads)).astype(np.float32)
        dy = np.random.default_rng(heads + 1).standard_normal((12, heads)).astype(np.float32)
        ti = torch.from_numpy(indptr).to(dev)
        for _ in range(2):   # a second call reuses freed memory that is not zero
            y = fa.forward_edge_softmax(ti, ti, torch.from_numpy(x).to(dev), 512, heads)[0]
            dx = fa.backward_edge_softmax(ti, ti, torch.from_numpy(dy).to(dev), y, 512, heads)[0]
        y_ref = C.edge_softmax_fwd(indptr, x, heads, 0)
        assert_rel(y, y_ref, 1e-6, f"forward, {heads} heads")
        assert not y[:3].any() and not y[9:].any()
        assert_rel(dx, C.edge_softmax_bwd(indptr, dy, y.cpu().numpy(), heads), 1e-6, "backward")
        assert not dx[:3].any() and not dx[9:].any()


# ---------------------------------------------------------------------------------------
# fused LeakyReLU + softmax + dropout + aggregation
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("p", [0.0, 0.3])
@pytest.mark.parametrize("H,dh", [(2, 50), (1, 127), (4, 32), (8, 7), (2, 100)])
@pytest.mark.parametrize("rows", ["own", "shared"])
def test_fused_attn(fa, dev, p, H, dh, rows):
    """Rows of up to 128 values take the half-wave kernels (odd widths the element loads),
    wider ones the one-wave kernels; degrees include 0, odd counts and more than 64. With
    every V row its own edge's (the sampler's layout) grad_V is stored row by row; V rows
    shared by several edges (and a source past n_src, ignored) take the atomic adds."""
    deg = DEGREE_SETS["ragged"]
    indptr, dst = _csr(deg)
    N, E = len(deg), dst.size
    rng = np.random.default_rng(7)
    if rows == "own":
        src = np.arange(N, N + E, dtype=np.int64)
    else:
        src = N + rng.integers(0, E // 3, E).astype(np.int64)
        src[5] = N + E + 3
    score = rng.standard_normal((E, H)).astype(np.float32)
    V = rng.standard_normal((E, H, dh)).astype(np.float32)
    dout = rng.standard_normal((N, H * dh)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    out, attn, mask = fa.forward_fused_attn(t(score), t(V), t(indptr), t(indptr), t(dst), t(src),
                                            N, H, 0.2, p)
    out_ref, attn_ref = C.fused_attn_fwd(indptr, dst, src, N, score, V, 0.2, p, mask.cpu().numpy())
    assert_rel(attn, attn_ref, 1e-6, "fused attn")
    assert_rel(out, out_ref, FP32_TOL, "fused out")
    d_act, gV = fa.backward_fused_attn(t(dout), t(V), attn, mask, t(indptr), t(indptr), t(dst),
                                       t(src), N + E, H, 0.2, p)
    d_ref, gV_ref = C.fused_attn_bwd(indptr, dst, src, N, N + E, dout, V, attn.cpu().numpy(),
                                     mask.cpu().numpy(), p)
    assert_rel(d_act, d_ref, FP32_TOL, "fused d_act")
    assert_rel(gV, gV_ref, FP32_TOL, "fused grad_V")


@pytest.mark.parametrize("case", ["offset", "bad_dst", "bad_src", "decreasing", "no_segments"])
@pytest.mark.parametrize("dh", [50, 127, 100])
def test_fused_attn_bwd_writes_every_row(fa, dev, case, dh):
    """backward_fused_attn's grad_V comes back without a prior zero fill: with each V row
    its own edge's, rows are stored once, zeros for the edges before the first segment and
    after the last, for segments whose destination is out of range and for edges whose
    source is out of range; offsets that decrease turn the row stores off (atomic adds into
    zeros). The memory handed back was filled with NaN by an earlier tensor, so a row left
    unwritten shows."""
    H = 2
    deg = [3, 0, 5, 2, 7, 1, 4, 9]
    indptr, dst = _csr(deg)
    N = len(deg)
    lead, trail = (3, 4) if case == "offset" else (0, 0)
    E = lead + dst.size + trail
    indptr = (indptr + lead).astype(np.int32)
    dst = np.concatenate([np.zeros(lead, np.int64), dst, np.zeros(trail, np.int64)])
    src = np.arange(N, N + E, dtype=np.int64)
    if case == "bad_dst":
        dst[indptr[1]:indptr[2]] = -1       # the second non-empty segment's destination
        dst[indptr[3]:indptr[4]] = N + 5
    elif case == "bad_src":
        src[4] = N + E + 3                  # past n_src
        src[9] = 2                          # below n_dst
    elif case == "decreasing":
        indptr = np.concatenate([indptr[:4], [2]]).astype(np.int32)
    elif case == "no_segments":
        indptr = indptr[:1]
    rng = np.random.default_rng(dh + len(case))
    score = rng.standard_normal((E, H)).astype(np.float32)
    V = rng.standard_normal((E, H, dh)).astype(np.float32)
    dout = rng.standard_normal((N, H * dh)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    out, attn, mask = fa.forward_fused_attn(t(score), t(V), t(indptr), t(indptr), t(dst), t(src),
                                            N, H, 0.2, 0.3)
    d_ref, gV_ref = C.fused_attn_bwd(indptr, dst, src, N, N + E, dout, V, attn.cpu().numpy(),
                                     mask.cpu().numpy(), 0.3)
    for _ in range(2):
        junk = torch.full((E * H * dh + 4096,), float("nan"), device=dev)
        del junk
        d_act, gV = fa.backward_fused_attn(t(dout), t(V), attn, mask, t(indptr), t(indptr),
                                           t(dst), t(src), N + E, H, 0.2, 0.3)
        assert torch.isfinite(gV).all(), "grad_V rows left unwritten"
        assert_rel(gV, gV_ref, FP32_TOL, f"grad_V {case}")
        assert_rel(d_act, d_ref, FP32_TOL, f"d_act {case}")


def test_inputs_must_be_on_gpu(fa):
    x = torch.zeros(4, 2)
    ip = torch.tensor([0, 2, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fa.forward_edge_softmax(ip, ip, x, 512, 2)
