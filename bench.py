"""Benchmark: temporal-attention aggregated edges/s, forward + backward, fanout 10, on one GPU.

One step = one training step of a 2-layer TGAT attention stack (modules.py:48-64 with the
layers of layers.py:53-240) over one synthetic MFG of config C3: 4000 roots x 3 = 12000
top-layer destinations, fanout [10, 10] (bottom block 132000 destinations / 1.32M edges, top
block 12000 / 120000), node rows gathered from a 1M x 100 table and edge rows from a
10M x 172 table by uniform random ids, dt ~ Exp(mean 1e4), time dim 100, 2 heads, hidden
100, float32, dropout 0.1 / attention dropout 0.1 (config/TGAT.yml), Adam. Inputs are
resident in HBM before timing; the step covers everything from the blocks' row offsets to
the optimizer update.

Prints one JSON line (see keys below). ``roofline`` is the fused kernel with the largest
total time, timed by HIP events around each launch; ``cpu_baseline`` is the CPU
restatement in oracle/ timed on the host cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "temporal-attn aggregated edges/s fwd+bwd (fanout 10); HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
# rocprofv3 --pmc summary of this workload (FETCH_SIZE / WRITE_SIZE per dispatch, scaled by
# the same counters on the copy probe below); gives roofline.traffic when present
PMC_SUMMARY = os.path.join(ROOT, "profiles", "tgat_C3_pmc_traffic.md")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--roots", type=int, default=4000)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-roots", type=int, default=4000,
                    help="roots of the bounded CPU sample (same MFG shape, fewer roots)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--config", choices=("c3", "c5"), default="c3",
                    help="c3: the headline float32 workload; c5: bf16 tables of widths 413 / 186 "
                         "(5M and 50M rows, 80%% of ids from a 5%% hot set), 8 heads, hidden 256")
    ap.add_argument("--dropin", action="store_true",
                    help="instead of the training step, time each drop-in fastAgg operator on the "
                         "ragged config (one JSON line per operator)")
    ap.add_argument("--copy-probe-mb", type=int, default=256,
                    help="after the timed steps, one plain row copy of this many MiB "
                         "(fastAgg.gather_rows over rows of 1024 floats): the known-size kernel "
                         "that scales the PMC byte counters; 0 disables it")
    return ap.parse_args()


def progress(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` (read + written) from the committed rocprofv3
    --pmc summary, or None when there is none for it."""
    try:
        with open(PMC_SUMMARY) as fh:
            text = fh.read()
    except OSError:
        return None
    m = re.search(rf"^traffic_per_launch\s+{re.escape(kernel)}\s+(\d+)\s*$", text, re.M)
    return int(m.group(1)) if m else None


def copy_probe(mb: int) -> None:
    """One row copy of ``mb`` MiB: reads mb MiB of rows + 8 B of index per row, writes mb MiB."""
    import torch

    import fast_amd

    rows = mb * 256  # 1024 floats = 4 KiB per row
    src = torch.randn(rows, 1024, device="cuda:0")
    idx = torch.arange(rows, device="cuda:0")
    torch.cuda.synchronize()
    fast_amd.fastAgg.gather_rows(src, idx, rows)
    torch.cuda.synchronize()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(roots: int, reps: int, seed: int) -> dict:
    """The CPU restatement (oracle/ref_cpu.py, float32, torch on the host cores) of the same
    2-layer forward + backward on a bounded sample: ``roots`` roots instead of 4000."""
    import torch

    from fast_amd.tgat import TGATEncoder
    from fast_amd.workloads import two_layer
    from oracle.ref_cpu import layer_params, tgat_layer

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(seed)
    enc = TGATEncoder(100, 172, 100, 2, 100, num_layers=2, dropout=0.0, att_dropout=0.0)
    inp = two_layer(roots=roots, n_nodes=1_000_000, n_edge_rows=1_000_000, seed=seed,
                    device="cpu")
    b0, b1 = inp.blocks
    s0, d0 = b0.edges()
    s1, d1 = b1.edges()

    def step():
        P0 = {k: (v.float().detach().requires_grad_(True) if isinstance(v, torch.Tensor) else v)
              for k, v in layer_params(enc.layers["l0h0"]).items()}
        P1 = {k: (v.float().detach().requires_grad_(True) if isinstance(v, torch.Tensor) else v)
              for k, v in layer_params(enc.layers["l1h0"]).items()}
        h0 = b0.node_table[b0.srcdata["ID"]]
        f0 = b0.edge_table[b0.edata["ID"]]
        r0 = tgat_layer(P0, h0, f0, b0.edata["dt"], s0, d0, b0.num_dst_nodes(), dtype=torch.float32)
        f1 = b1.edge_table[b1.edata["ID"]]
        r1 = tgat_layer(P1, r0, f1, b1.edata["dt"], s1, d1, b1.num_dst_nodes(), dtype=torch.float32)
        r1.backward(inp.dout)

    step()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    t = times[len(times) // 2]
    edges = sum(inp.edges_per_layer)
    return {"value": edges / t, "unit": "edges/s", "cores": cores, "kind": "port",
            "sample": (f"2-layer TGAT fwd+bwd, {roots} roots x3 (blocks {b0.num_dst_nodes()}/"
                       f"{inp.edges_per_layer[0]} and {b1.num_dst_nodes()}/{inp.edges_per_layer[1]}"
                       f" dst/edges), float32, median of {reps} after 1 warm-up: "
                       f"{t * 1e3:.1f} ms/step; CPU: {cpu_model()}")}


def dropin_bench(reps: int = 20, seed: int = 0) -> None:
    """Each drop-in operator (operators.cpp:606-625 names) on the ragged config C4: 200000
    destinations, Zipf(1.5) degrees clipped to [1, 20], 5 % empty; 2 heads, D = 100 (dh 50).
    Prints per operator the average call time (HIP events around the binding call, output
    allocation and zero fill included) and its algorithmic bytes / time."""
    import numpy as np
    import torch

    import fast_amd
    from fast_amd.workloads import ragged_degrees

    fa = fast_amd.fastAgg
    dev = torch.device("cuda:0")
    deg = ragged_degrees(200_000, seed)
    N, E, H, D = deg.size, int(deg.sum()), 2, 100
    nz = deg[deg > 0]
    S = nz.size
    g = torch.Generator(device=dev).manual_seed(seed)
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(nz)]).astype(np.int32)).to(dev)
    dst = torch.from_numpy(np.repeat(np.arange(N), deg)).to(dev)
    src = torch.arange(N, N + E, device=dev)
    x = torch.randn(E, H, device=dev, generator=g)
    y = fa.forward_edge_softmax(indptr, indptr, x, 512, H)[0]
    feat = torch.randn(N + E, D, device=dev, generator=g)
    dout = torch.randn(N, D, device=dev, generator=g)
    V = torch.randn(E, H, D // H, device=dev, generator=g)
    out, attn, mask = fa.forward_fused_attn(x, V, indptr, indptr, dst, src, N, H, 0.2, 0.1)
    deg32 = torch.from_numpy(nz.astype(np.int32)).to(dev)
    ids32 = dst.to(torch.int32)
    cases = [
        ("forward_edge_softmax", lambda: fa.forward_edge_softmax(indptr, indptr, x, 512, H), 8 * E * H + 4 * (S + 1)),
        ("backward_edge_softmax", lambda: fa.backward_edge_softmax(indptr, indptr, x, y, 512, H), 12 * E * H + 4 * (S + 1)),
        ("forward_csr_edge_softmax", lambda: fa.forward_csr_edge_softmax(indptr, indptr, x, 32, 16), 8 * E * H + 4 * (S + 1)),
        ("backward_csr_edge_softmax", lambda: fa.backward_csr_edge_softmax(indptr, indptr, x, y, 32, 16), 12 * E * H + 4 * (S + 1)),
        ("forward_tgat", lambda: fa.forward_tgat(dst, src, feat, N, 8, 128), 16 * E + 4 * E * D + 4 * N * D),
        ("backward_tgat", lambda: fa.backward_tgat(dst, src, dout, N + E, 8, 128), 16 * E + 8 * E * D),
        ("forward_tgat_shd", lambda: fa.forward_tgat_shd(indptr, indptr, dst, src, feat, N, 8, 32), 4 * (S + 1) + 16 * E + 4 * E * D + 4 * N * D),
        ("backward_tgat_shd", lambda: fa.backward_tgat_shd(indptr, indptr, dst, src, dout, N + E, 8, 32), 4 * (S + 1) + 16 * E + 8 * E * D),
        ("forward_fused_attn", lambda: fa.forward_fused_attn(x, V, indptr, indptr, dst, src, N, H, 0.2, 0.1), 16 * E + 4 * E * D + 16 * E * H + 4 * N * D),
        ("backward_fused_attn", lambda: fa.backward_fused_attn(dout, V, attn, mask, indptr, indptr, dst, src, N + E, H, 0.2, 0.1), 16 * E + 8 * E * D + 16 * E * H + 4 * N * D),
        ("exclusive_sum", lambda: fa.exclusive_sum(deg32), 8 * S + 4),
        ("cal_deg", lambda: fa.cal_deg(ids32, N), 4 * E + 4 * N),
        ("getBalancedPtr", lambda: fa.getBalancedPtr(indptr, 16), 8 * S),
    ]
    for name, fn, nbytes in cases:
        fn()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            fn()
        s1.record()
        torch.cuda.synchronize()
        us = s0.elapsed_time(s1) * 1e3 / reps
        print(json.dumps({"op": name, "workload": f"C4 ragged: N={N}, S={S}, E={E}, H={H}, D={D}",
                          "call_us": round(us, 2), "algorithmic_bytes": nbytes,
                          "GB/s": round(nbytes / us / 1e3, 1),
                          "frac_of_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)


def main():
    args = parse()
    if args.dropin:
        if args.gpus != 1:
            print("bench.py: this build runs on one GPU only", file=sys.stderr)
            sys.exit(2)
        dropin_bench()
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding is design-only (DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch

    import fast_amd
    from fast_amd import tgat
    from fast_amd.tgat import TGATEncoder
    from fast_amd.workloads import two_layer

    dev = torch.device("cuda:0")
    # rocBLAS picks faster fp32 kernels than hipBLASLt for the layer's tall-skinny
    # projections ([N, 100] x [100, 752] and transposes) on this stack
    torch.backends.cuda.preferred_blas_library("cublas")
    torch.manual_seed(args.seed)
    if args.config == "c5":
        dims = (413, 186, 100, 8, 256)
        enc = TGATEncoder(*dims, num_layers=2, dropout=0.1, att_dropout=0.1).to(dev)
        inp = two_layer(roots=args.roots, n_nodes=5_000_000, n_edge_rows=50_000_000, dn=413,
                        de=186, heads=8, dim_out=256, seed=args.seed, device=dev, hot_frac=0.05,
                        hot_share=0.8, dtype=torch.bfloat16, row_align=4)
        desc = ("C5: 2-layer TGAT attention fwd+bwd+Adam, bf16 tables (rows padded to 416 / 188), "
                "node table 5M x 413, edge table 50M x 186, 80% of ids from a 5% hot set, time 100, "
                "8 heads, hidden 256")
        dtype = "bf16 tables, f32 compute"
    else:
        enc = TGATEncoder(100, 172, 100, 2, 100, num_layers=2, dropout=0.1, att_dropout=0.1).to(dev)
        inp = two_layer(roots=args.roots, seed=args.seed, device=dev)
        desc = ("C3: 2-layer TGAT attention fwd+bwd+Adam, node table 1M x 100, edge table "
                "10M x 172, time 100, 2 heads, hidden 100")
        dtype = "f32"
    enc.train()
    # one fused multi-tensor kernel for the update (the foreach form launches seven)
    opt = torch.optim.Adam(enc.parameters(), lr=1e-4, fused=True)
    blocks = inp.blocks
    edges = sum(inp.edges_per_layer)

    def step():
        for b in blocks:
            b._rowptr = None  # a new batch's offsets are derived inside the step
        opt.zero_grad(set_to_none=True)
        out = enc(blocks)
        out.backward(inp.dout)
        opt.step()

    progress(f"inputs resident: {len(blocks)} blocks, {edges} edges per step")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    progress(f"{args.warmup} warm-up steps done")
    timer = tgat.KernelTimer()
    tgat.timer = timer
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    tgat.timer = None
    progress(f"{args.steps} timed steps done: {(t1 - t0) * 1e3 / args.steps:.3f} ms/step")
    if args.copy_probe_mb > 0:
        copy_probe(args.copy_probe_mb)
    ms = (t1 - t0) * 1e3 / args.steps
    kern = timer.summary()
    dom_name = max(kern, key=lambda k: kern[k]["ms"])
    dom = kern[dom_name]
    fused_ms = sum(d["ms"] for d in kern.values()) / args.steps

    line = {
        "metric": METRIC,
        "value": edges / (ms * 1e-3),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded N(0,1) tables, uniform ids, Exp(1e4) dt; random-init weights)",
        "config": {
            "workload": (f"{desc}; {args.roots} roots x3, fanout [10,10], blocks "
                         f"{blocks[0].num_dst_nodes()}/{inp.edges_per_layer[0]} and "
                         f"{blocks[1].num_dst_nodes()}/{inp.edges_per_layer[1]} dst/edges"),
            "edges_per_step": edges,
            "fused_kernel_edges_per_s": edges / (fused_ms * 1e-3),
            "fused_kernels_ms_per_step": fused_ms,
            "kernels": {k: {"launches": v["launches"], "avg_us": round(v["avg_us"], 2),
                            "GB/s": round(v["GB/s"], 1)} for k, v in kern.items()},
        },
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": dom["GB/s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["GB/s"] / HBM_PEAK_GBS,
            "traffic": measured_traffic(dom_name) if args.config == "c3" else None,
            "algorithmic_bytes_per_launch": dom["bytes"] // max(1, dom["launches"]),
        },
    }
    if not args.no_cpu_baseline and args.config == "c3":
        line["cpu_baseline"] = cpu_baseline(args.cpu_roots, args.cpu_reps, args.seed)
        progress("cpu baseline done")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
