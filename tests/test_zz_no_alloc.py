"""The fused backward's no-allocation entry point (fa_tgat_attn_bwd_noalloc_f32, whose
time-gradient partials live in the library's static device array) against the entry point
that takes caller scratch (fa_tgat_attn_bwd_f32), both called through the C ABI: equal
outputs, bit for bit, on two calls in a row, the second on a smaller graph (fewer
workgroups, so rows the first call left in the array must not be read)."""
import ctypes

import pytest
import torch

from tests.test_abi import TgatGraph

pytestmark = pytest.mark.gpu


def _lib():
    import fast_amd

    lib = ctypes.CDLL(fast_amd.lib_path())
    lib.fa_tgat_attn_bwd_scratch_bytes.restype = ctypes.c_size_t
    return lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _case(dev, N, H, dn, de, dtd, max_deg, seed, drop_p):
    """A random graph with gathered tables, its forward outputs (fastAgg binding) and the
    backward's inputs."""
    from fast_amd import fastAgg
    from fast_amd.tgat import kspace_width

    g = torch.Generator().manual_seed(seed)
    deg = torch.randint(0, max_deg + 1, (N,), generator=g)
    rowptr = torch.zeros(N + 1, dtype=torch.int32)
    rowptr[1:] = torch.cumsum(deg, 0).to(torch.int32)
    E = int(rowptr[-1])
    kp = kspace_width(dn, de, dtd)
    t = dict(rowptr=rowptr, ntab=torch.randn(700, dn, generator=g),
             nid=torch.randint(0, 700, (E,), generator=g),
             etab=torch.randn(1500, de, generator=g),
             eid=torch.randint(0, 1500, (E,), generator=g),
             dt=torch.empty(E).exponential_(1e-4, generator=g),
             tw=torch.randn(dtd, generator=g) * 0.1, tb=torch.randn(dtd, generator=g),
             qt=torch.randn(H, N, kp, generator=g) * 0.05,
             dxbar=torch.randn(H, N, kp, generator=g))
    t = {k: v.to(dev) for k, v in t.items()}
    xbar, scores, stats = fastAgg.tgat_attn_fwd(t["rowptr"], t["ntab"], t["nid"], t["etab"],
                                                t["eid"], t["dt"], t["tw"], t["tb"], t["qt"],
                                                0.2, None, 1234, drop_p)
    t.update(xbar=xbar, scores=scores, stats=stats, E=E, kp=kp, N=N, H=H, dn=dn, dtd=dtd)
    graph = TgatGraph(n_dst=N, n_edges=E, rowptr=t["rowptr"].data_ptr(),
                      node_tab=t["ntab"].data_ptr(), ld_node=dn, n_node=700, dn=dn,
                      node_idx=t["nid"].data_ptr(), node_dtype=0,
                      edge_tab=t["etab"].data_ptr(), ld_edge=de, n_edge_rows=1500, de=de,
                      edge_idx=t["eid"].data_ptr(), edge_dtype=0, dt=t["dt"].data_ptr(),
                      time_w=t["tw"].data_ptr(), time_b=t["tb"].data_ptr(), dt_dim=dtd)
    return graph, t


def _bwd(lib, graph, t, drop_p, noalloc):
    """One backward through the C ABI; returns (dqt, d_node, d_time_w, d_time_b)."""
    dev = t["qt"].device
    N, H, kp, E = t["N"], t["H"], t["kp"], t["E"]
    dqt = torch.full((H, N, kp), float("nan"), device=dev)
    d_node = torch.full((E, t["dn"]), float("nan"), device=dev)
    dtw = torch.full((t["dtd"],), float("nan"), device=dev)
    dtb = torch.full((t["dtd"],), float("nan"), device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    x = t["xbar"]
    args = [ctypes.byref(graph), ctypes.c_int32(H), _ptr(t["qt"]), ctypes.c_int64(kp),
            ctypes.c_int64(N * kp), ctypes.c_float(0.2), None, ctypes.c_uint64(1234),
            ctypes.c_float(drop_p), _ptr(x), ctypes.c_int64(x.stride(1)),
            ctypes.c_int64(x.stride(0)), None, _ptr(t["scores"]), _ptr(t["stats"]),
            _ptr(t["dxbar"]), ctypes.c_int64(kp), ctypes.c_int64(N * kp), _ptr(dqt),
            ctypes.c_int64(kp), ctypes.c_int64(N * kp), _ptr(d_node), ctypes.c_int64(t["dn"]),
            _ptr(dtw), _ptr(dtb)]
    if noalloc:
        st = lib.fa_tgat_attn_bwd_noalloc_f32(*args, stream)
    else:
        sb = lib.fa_tgat_attn_bwd_scratch_bytes(ctypes.c_int64(N), ctypes.c_int32(t["dtd"]))
        scratch = torch.full((max(1, sb // 4),), float("nan"), device=dev)
        st = lib.fa_tgat_attn_bwd_f32(*args, _ptr(scratch), ctypes.c_size_t(sb), stream)
    assert st == 0, st
    torch.cuda.synchronize(dev)
    return dqt, d_node, dtw, dtb


def test_noalloc_backward_matches_scratch_entry(dev):
    lib = _lib()
    # a large graph (two heads: the two-edge backward, many workgroups), then a smaller one
    # (eight heads, unaligned node rows: the one-edge backward, fewer workgroups)
    cases = [dict(N=6000, H=2, dn=100, de=172, dtd=100, max_deg=25, seed=1, drop_p=0.1),
             dict(N=300, H=8, dn=13, de=6, dtd=9, max_deg=12, seed=2, drop_p=0.0)]
    for c in cases:
        print(f"[no-alloc] case {c}", flush=True)
        graph, t = _case(dev, c["N"], c["H"], c["dn"], c["de"], c["dtd"], c["max_deg"], c["seed"],
                         c["drop_p"])
        want = _bwd(lib, graph, t, c["drop_p"], noalloc=False)
        got = _bwd(lib, graph, t, c["drop_p"], noalloc=True)
        for a, b, name in zip(got, want, ("dqt", "d_node", "d_time_w", "d_time_b")):
            assert not torch.isnan(b).any(), name
            assert torch.equal(a, b), f"{name} differs (case {c})"
