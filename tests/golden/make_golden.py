"""Writes the golden fixtures that pin the CPU restatement in oracle/.

The FAST reference ships no tests, fixtures or golden vectors, and its path cannot be
imported here (it needs dgl and the CUDA fastAgg build). These fixtures are therefore
computed from the definitions with plain Python loops over floats (math.exp / math.cos in
double precision, no numpy linear algebra, no torch, nothing from oracle/), on small seeded
inputs, so that an index, sign, operand-order or concatenation-order mistake in the oracle
shows up as a mismatch.

Run: python tests/golden/make_golden.py   (rewrites tests/golden/*.json)
"""
from __future__ import annotations

import json
import math
import os
import random

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(x: float) -> float:
    return float(np.float32(x))


def wrap32(x: int) -> int:
    return ((x + 2**31) % 2**32) - 2**31


def trunc_div(a: int, b: int) -> int:
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b > 0) else -q


# -------------------------------------------------------------------------------------
# bookkeeping (utils.cu:16-141, sampler_core.cpp:384-409)
# -------------------------------------------------------------------------------------
def bookkeeping(rng: random.Random) -> dict:
    cases = {"exclusive_sum": [], "cal_deg": [], "balance_mask": [], "rowptr": [], "cnte": []}
    for n in (0, 1, 5, 300):
        x = [rng.randint(0, 9) for _ in range(n)]
        out, acc = [0], 0
        for v in x:
            acc = wrap32(acc + v)
            out.append(acc)
        cases["exclusive_sum"].append({"in": x, "out": out})
    big = [2**30] * 5
    out, acc = [0], 0
    for v in big:
        acc = wrap32(acc + v)
        out.append(acc)
    cases["exclusive_sum"].append({"in": big, "out": out})
    for n_ids, n_nodes in ((0, 3), (40, 6), (200, 17)):
        ids = [rng.randint(-2, n_nodes + 1) for _ in range(n_ids)]
        deg = [0] * n_nodes
        for v in ids:
            if 0 <= v < n_nodes:
                deg[v] += 1
        cases["cal_deg"].append({"ids": ids, "n_nodes": n_nodes, "out": deg})
    for n, thr in ((1, 3), (9, 4), (600, 7), (520, -3)):
        ptr = [0]
        for _ in range(n - 1):
            ptr.append(ptr[-1] + rng.randint(0, 15))
        mask = []
        for i in range(n - 1):
            blk = (i // 256) * 256
            p_after = sum(ptr[j + 1] - ptr[j] for j in range(blk, i + 1))
            p_before = p_after - (ptr[i + 1] - ptr[i])
            mask.append(1 if trunc_div(p_after, thr) > trunc_div(p_before, thr) else 0)
        cases["balance_mask"].append({"ptr": ptr, "threshold": thr, "out": mask})
    for degs in ([3, 0, 2, 0, 0, 1], [0, 0], [5]):
        dst = [v for v, d in enumerate(degs) for _ in range(d)]
        rowptr = [sum(degs[:v]) for v in range(len(degs) + 1)]
        cases["rowptr"].append({"dst": dst, "n_dst": len(degs), "out": rowptr})
        # sampler cntE: run lengths of the sorted row array, cumulated, starting at 0
        cnte, run = [0], 0
        for i, r in enumerate(dst):
            run += 1
            if i + 1 == len(dst) or dst[i + 1] != r:
                cnte.append(cnte[-1] + run)
                run = 0
        cases["cnte"].append({"dst": dst, "out": cnte})
    return cases


# -------------------------------------------------------------------------------------
# softmax / aggregation (edge_softmax.cu:255-329, aggregate_*.cu, fused_attention.cu)
# -------------------------------------------------------------------------------------
def softmax_cases(rng: random.Random) -> list:
    out = []
    for degs, heads in (([1, 2, 3, 0, 5], 2), ([10] * 4, 1), ([17, 20], 8), ([2, 2], 2)):
        indptr = [0]
        for d in degs:
            if d:
                indptr.append(indptr[-1] + d)
        E = indptr[-1]
        x = [[f32(rng.gauss(0, 3)) for _ in range(heads)] for _ in range(E)]
        if degs == [2, 2]:
            x = [[1.5, -2.0], [1.5, -2.0], [0.0, 80.0], [0.0, -80.0]]  # ties; large gap
        dy = [[f32(rng.gauss(0, 1)) for _ in range(heads)] for _ in range(E)]
        y = [[0.0] * heads for _ in range(E)]
        dx = [[0.0] * heads for _ in range(E)]
        for s in range(len(indptr) - 1):
            lb, le = indptr[s], indptr[s + 1]
            for h in range(heads):
                m = max(x[e][h] for e in range(lb, le))
                z = sum(math.exp(x[e][h] - m) for e in range(lb, le))
                for e in range(lb, le):
                    y[e][h] = math.exp(x[e][h] - m) / z
                t = sum(y[e][h] * dy[e][h] for e in range(lb, le))
                for e in range(lb, le):
                    dx[e][h] = y[e][h] * (dy[e][h] - t)
        out.append({"indptr": indptr, "heads": heads, "x": x, "dy": dy, "y": y, "dx": dx})
    return out


def aggregation_cases(rng: random.Random) -> list:
    out = []
    for degs, dim in (([2, 0, 3, 1], 3), ([1] * 5, 1), ([4, 4], 2)):
        N = len(degs)
        dst = [v for v, d in enumerate(degs) for _ in range(d)]
        E = len(dst)
        src = list(range(N, N + E))
        x = [[f32(rng.gauss(0, 1)) for _ in range(dim)] for _ in range(N + E)]
        dout = [[f32(rng.gauss(0, 1)) for _ in range(dim)] for _ in range(N)]
        agg = [[0.0] * dim for _ in range(N)]
        for e in range(E):
            for c in range(dim):
                agg[dst[e]][c] += x[src[e]][c]
        dx = [[0.0] * dim for _ in range(N + E)]
        for e in range(E):
            for c in range(dim):
                dx[src[e]][c] += dout[dst[e]][c]
        indptr = [0]
        for d in degs:
            if d:
                indptr.append(indptr[-1] + d)
        out.append({"dst": dst, "src": src, "x": x, "dout": dout, "n_dst": N, "indptr": indptr,
                    "agg": agg, "dx": dx})
    return out


def fused_attn_case(rng: random.Random) -> dict:
    degs, H, dh, p, slope = [3, 0, 2, 4], 2, 3, 0.25, 0.2
    N = len(degs)
    dst = [v for v, d in enumerate(degs) for _ in range(d)]
    E = len(dst)
    src = list(range(N, N + E))
    indptr = [0]
    for d in degs:
        if d:
            indptr.append(indptr[-1] + d)
    score = [[f32(rng.gauss(0, 2)) for _ in range(H)] for _ in range(E)]
    V = [[[f32(rng.gauss(0, 1)) for _ in range(dh)] for _ in range(H)] for _ in range(E)]
    mask = [[f32(rng.random()) for _ in range(H)] for _ in range(E)]
    dout = [[f32(rng.gauss(0, 1)) for _ in range(H * dh)] for _ in range(N)]
    lk = lambda z: z if z > 0 else z * slope
    attn = [[0.0] * H for _ in range(E)]
    out = [[0.0] * (H * dh) for _ in range(N)]
    d_act = [[0.0] * H for _ in range(E)]
    gV = [[[0.0] * dh for _ in range(H)] for _ in range(E)]
    for v in range(N):
        es = [e for e in range(E) if dst[e] == v]
        if not es:
            continue
        for h in range(H):
            m = max(lk(score[e][h]) for e in es)
            z = sum(math.exp(lk(score[e][h]) - m) for e in es)
            for e in es:
                attn[e][h] = math.exp(lk(score[e][h]) - m) / z
            da = {}
            for e in es:
                keep = 1 / (1 - p) if mask[e][h] > p else 0.0
                for d in range(dh):
                    out[v][h * dh + d] += attn[e][h] * keep * V[src[e] - N][h][d]
                    gV[src[e] - N][h][d] += attn[e][h] * keep * dout[v][h * dh + d]
                da[e] = keep * sum(dout[v][h * dh + d] * V[src[e] - N][h][d] for d in range(dh))
            t = sum(attn[e][h] * da[e] for e in es)
            for e in es:
                d_act[e][h] = attn[e][h] * (da[e] - t)
    return {"indptr": indptr, "dst": dst, "src": src, "n_dst": N, "score": score, "V": V,
            "mask": mask, "p": p, "slope": slope, "dout": dout, "attn": attn, "out": out,
            "d_act": d_act, "grad_V": gV}


# -------------------------------------------------------------------------------------
# one TGAT layer (layers.py:98-240, TGAT branch, DGL semantics)
# -------------------------------------------------------------------------------------
def layer_norm(row, w, b, eps):
    n = len(row)
    mu = sum(row) / n
    var = sum((r - mu) ** 2 for r in row) / n
    return [(r - mu) / math.sqrt(var + eps) * w[i] + b[i] for i, r in enumerate(row)]


def linear(x, W, b):
    return [sum(W[o][i] * x[i] for i in range(len(x))) + b[o] for o in range(len(W))]


def tgat_forward(P, h, f, dt, dst, N, H, slope=0.2, eps=1e-5, round_arg=True):
    """Forward of the layer with plain loops. P: dict of nested lists. With round_arg the
    time-encoding argument is rounded like the float32 reference; without it the argument
    is exact (used for finite differences, whose steps are below a float32 ulp)."""
    E = len(dst)
    Dt = len(P["tw"])
    D = len(P["bq"])
    dh = D // H

    def tenc(t):
        # argument rounded as the float32 Linear(1, Dt) result: product, then sum
        if round_arg:
            return [math.cos(f32(f32(t * P["tw"][j]) + P["tb"][j])) for j in range(Dt)]
        return [math.cos(t * P["tw"][j] + P["tb"][j]) for j in range(Dt)]

    Q = [linear(h[v] + tenc(0.0), P["Wq"], P["bq"]) for v in range(N)]
    K, Vv = [], []
    for e in range(E):
        kv = h[N + e] + f[e] + tenc(dt[e])
        K.append(linear(kv, P["Wk"], P["bk"]))
        Vv.append(linear(kv, P["Wv"], P["bv"]))
    lk = lambda z: z if z > 0 else z * slope
    sc = [[lk(sum(Q[dst[e]][hh * dh + d] * K[e][hh * dh + d] for d in range(dh)))
           for hh in range(H)] for e in range(E)]
    agg = [[0.0] * D for _ in range(N)]
    for v in range(N):
        es = [e for e in range(E) if dst[e] == v]
        for hh in range(H):
            if not es:
                continue
            m = max(sc[e][hh] for e in es)
            z = sum(math.exp(sc[e][hh] - m) for e in es)
            for e in es:
                a = math.exp(sc[e][hh] - m) / z
                for d in range(dh):
                    agg[v][hh * dh + d] += a * Vv[e][hh * dh + d]
    out = []
    for v in range(N):
        r = linear(agg[v] + h[v], P["Wo"], P["bo"])
        r = [max(0.0, x) for x in r]
        out.append(layer_norm(r, P["lnw"], P["lnb"], eps))
    return out


def tgat_case(rng: random.Random) -> dict:
    degs = [2, 0, 3, 1]
    Dn, De, Dt, H, D = 2, 3, 2, 2, 4
    N = len(degs)
    dst = [v for v, d in enumerate(degs) for _ in range(d)]
    E = len(dst)
    g = lambda s=1.0: f32(rng.gauss(0, s))
    mat = lambda r, c, s: [[g(s) for _ in range(c)] for _ in range(r)]
    P = {
        "tw": [f32(1 / 10 ** (9 * j / (Dt - 1))) for j in range(Dt)],
        "tb": [f32(0.3), f32(-1.1)],
        "Wq": mat(D, Dn + Dt, 0.5), "bq": [g(0.1) for _ in range(D)],
        "Wk": mat(D, Dn + De + Dt, 0.5), "bk": [g(0.1) for _ in range(D)],
        "Wv": mat(D, Dn + De + Dt, 0.5), "bv": [g(0.1) for _ in range(D)],
        "Wo": mat(D, Dn + D, 0.5), "bo": [g(0.1) for _ in range(D)],
        "lnw": [f32(1 + g(0.1)) for _ in range(D)], "lnb": [g(0.1) for _ in range(D)],
    }
    h = mat(N + E, Dn, 1.0)
    f = mat(E, De, 1.0)
    dt = [f32(rng.expovariate(1e-4)) for _ in range(E)]
    out = tgat_forward(P, h, f, dt, dst, N, H)
    # central finite differences of sum(out * W) for a few scalars (double precision)
    wsum = mat(N, D, 1.0)

    def loss(Pm, hm):
        o = tgat_forward(Pm, hm, f, dt, dst, N, H, round_arg=False)
        return sum(o[v][i] * wsum[v][i] for v in range(N) for i in range(D))

    fd = {}
    step = 1e-6
    for key, idx in (("Wk", (1, 2)), ("Wv", (3, 6)), ("Wq", (0, 3)), ("tb", (1,)), ("tw", (0,)),
                     ("Wo", (2, 5)), ("bk", (1,)), ("h", (N + 1, 1)), ("h", (0, 0))):
        def perturb(delta):
            Pm = json.loads(json.dumps(P))
            hm = json.loads(json.dumps(h))
            tgt = hm if key == "h" else Pm[key]
            if len(idx) == 1:
                tgt[idx[0]] += delta
            else:
                tgt[idx[0]][idx[1]] += delta
            return loss(Pm, hm)
        scale = 1e-7 if key == "tw" else step
        fd[f"{key}{list(idx)}"] = (perturb(scale) - perturb(-scale)) / (2 * scale)
    return {"degs": degs, "dims": [Dn, De, Dt, H, D], "dst": dst, "P": P, "h": h, "f": f,
            "dt": dt, "out": out, "wsum": wsum, "fd_grads": fd}


def time_weight() -> dict:
    w = (1 / 10 ** np.linspace(0, 9, 100, dtype=np.float32)).astype(np.float32)
    exact = [10 ** (-9 * j / 99) for j in range(100)]
    return {"w_float32": [float(v) for v in w], "w_exact": exact}


def mfg_case() -> dict:
    """Sampler results (sampler_core.cpp layout: edges grouped by ascending destination
    `row`, edge e from source dim_out + e; some destinations without edges) and the blocks
    utils.py:67-87 to_dgl_blocks builds from them (dgl.create_block((src, dst)) with the
    roles of row / col set by `reverse`), grouped `hist` at a time with the incomplete last
    group dropped (zip(*[iter(x)] * hist)) and the groups reversed; plus the sampler's cntE
    (sampler_core.cpp:384-409: 0, then the running sum of the run lengths of `row`) and the
    full CSR over every destination. A generator of its own, so the other fixtures keep
    their values."""
    rng = random.Random(7001)
    results = []
    for dim_out in (4, 1, 6, 3, 5):
        degs = [rng.choice([0, 1, 2, 3, 5]) for _ in range(dim_out)]
        row = [v for v in range(dim_out) for _ in range(degs[v])]
        E = len(row)
        dim_in = dim_out + E
        results.append({
            "row": row, "col": [dim_out + e for e in range(E)],
            "nodes": [rng.randrange(10 ** 6) for _ in range(dim_in)],
            "dts": [f32(rng.random() * 1e4) for _ in range(dim_in)],
            "ts": [f32(rng.random() * 1e6) for _ in range(dim_in)],
            "eid": [rng.randrange(10 ** 7) for _ in range(E)],
            "dim_in": dim_in, "dim_out": dim_out})

    def blocks(reverse):
        out = []
        for r in results:
            if not reverse:
                b = {"src": r["col"], "dst": r["row"], "num_src": r["dim_in"], "num_dst": r["dim_out"],
                     "node_side": "src", "dt": r["dts"][r["dim_out"]:]}
            else:
                b = {"src": r["row"], "dst": r["col"], "num_src": r["dim_out"], "num_dst": r["dim_in"],
                     "node_side": "dst", "dt": r["dts"][r["dim_out"]:]}
            b.update(ID=r["nodes"], ts=r["ts"], eID=r["eid"])
            out.append(b)
        return out

    expect = {}
    for hist in (1, 2):
        for reverse in (False, True):
            bl = blocks(reverse)
            groups = [bl[g * hist:(g + 1) * hist] for g in range(len(bl) // hist)]
            groups.reverse()
            expect[f"hist{hist}_rev{int(reverse)}"] = groups
    cnte, rowptr = [], []
    for r in results:
        c, run = [0], 0
        for i, v in enumerate(r["row"]):
            run += 1
            if i + 1 == len(r["row"]) or r["row"][i + 1] != v:
                c.append(c[-1] + run)
                run = 0
        cnte.append(c)
        rowptr.append([sum(1 for v in r["row"] if v < d) for d in range(r["dim_out"] + 1)])
    return {"results": results, "blocks": expect, "cnte": cnte, "rowptr": rowptr}


# -------------------------------------------------------------------------------------
# TGN node memory (memorys.py:6-304)
# -------------------------------------------------------------------------------------
def sigmoid(x: float) -> float:
    return 1.0 / (1.0 + math.exp(-x))


def memory_case() -> dict:
    """MailBox.prep_input_mails (memorys.py:67-71), then two batches of update_mailbox
    ('self', 'last': memorys.py:113-139) followed by update_memory (memorys.py:86-103), in the
    order train.py:220-221 calls them, simulated row by row: the mails of edge k are
    [mem_src, mem_dst, ef] for its source and [mem_dst, mem_src, ef] for its destination,
    interleaved (source, destination, ...), the interleaved row r paired with ts[r]; per node
    the last row wins and writes slot next_mail_pos (advanced modulo the slot count when
    there is more than one slot); update_memory assigns rows 0..2n-1 in order. Roots repeat
    within and across batches. A generator of its own."""
    rng = random.Random(7002)
    cases = []
    for N, m, de, slots in ((12, 3, 2, 3), (9, 2, 0, 1)):
        mail = 2 * m + de
        st = {"node_memory": [[f32(rng.gauss(0, 1)) for _ in range(m)] for _ in range(N)],
              "node_memory_ts": [f32(rng.random() * 100) for _ in range(N)],
              "mailbox": [[[f32(rng.gauss(0, 1)) for _ in range(mail)] for _ in range(slots)]
                          for _ in range(N)],
              "mailbox_ts": [[f32(rng.random() * 100) for _ in range(slots)] for _ in range(N)],
              "next_mail_pos": [rng.randrange(slots) for _ in range(N)]}
        init = json.loads(json.dumps(st))
        ids = [rng.randrange(N) for _ in range(15)]
        prep = json.loads(json.dumps({
            "ids": ids,
            "mem": [st["node_memory"][i] for i in ids],
            "mem_ts": [st["node_memory_ts"][i] for i in ids],
            "mem_input": [[v for s_ in st["mailbox"][i] for v in s_] for i in ids],
            "mail_ts": [st["mailbox_ts"][i] for i in ids]}))   # a copy: the batches below
        # update the state's lists in place
        batches = []
        for _ in range(2):
            n, neg = 5, 1
            roots = [rng.randrange(N) for _ in range(n * (neg + 2))]
            n_rows = len(roots) + 4
            memory = [[f32(rng.gauss(0, 1)) for _ in range(m)] for _ in range(n_rows)]
            lu_nid = roots + [rng.randrange(N) for _ in range(4)]
            lu_ts = [f32(rng.random() * 1000) for _ in range(n_rows)]
            ts = [f32(rng.random() * 1000) for _ in range(len(roots))]
            ef = [[f32(rng.gauss(0, 1)) for _ in range(de)] for _ in range(n)]
            rows = []
            for k in range(n):
                rows.append((roots[k], memory[k] + memory[n + k] + ef[k], ts[2 * k]))
                rows.append((roots[n + k], memory[n + k] + memory[k] + ef[k], ts[2 * k + 1]))
            last = {}
            for r, (nid, _, _) in enumerate(rows):
                last[nid] = r
            for nid in sorted(last):
                _, ml, mt = rows[last[nid]]
                pos = st["next_mail_pos"][nid]
                st["mailbox"][nid][pos] = list(ml)
                st["mailbox_ts"][nid][pos] = mt
                if slots > 1:
                    st["next_mail_pos"][nid] = (pos + 1) % slots
            for i in range(len(roots) // (neg + 2) * 2):
                st["node_memory"][lu_nid[i]] = list(memory[i])
                st["node_memory_ts"][lu_nid[i]] = lu_ts[i]
            batches.append({"roots": roots, "neg": neg, "memory": memory, "nid": lu_nid,
                            "lu_ts": lu_ts, "ts": ts, "edge_feats": ef,
                            "after": json.loads(json.dumps(st))})
        cases.append({"dims": [N, m, de, slots], "init": init, "prep": prep, "batches": batches})
    return {"cases": cases}


def recurrent_case() -> dict:
    """GRUMemeoryUpdater / RNNMemeoryUpdater forward (memorys.py:286-293, 322-329) on three
    rows: x = [mails, cos(w (ts - mem_ts) + b)] with the time argument rounded as the
    reference's float32 Linear(1, dt) rounds it, then torch.nn.GRUCell's equations with gate
    blocks (r, z, n): r = s(W_ir x + b_ir + W_hr h + b_hr), z likewise, n = tanh(W_in x +
    b_in + r (W_hn h + b_hn)), h' = (1 - z) n + z h; and RNNCell's h' = tanh(W_ih x + b_ih +
    W_hh h + b_hh)."""
    rng = random.Random(7003)
    rows, mail, dt, hid = 3, 4, 3, 2
    din = mail + dt
    g = lambda: f32(rng.gauss(0, 0.5))
    P = {"w_ih": [[g() for _ in range(din)] for _ in range(3 * hid)],
         "w_hh": [[g() for _ in range(hid)] for _ in range(3 * hid)],
         "b_ih": [g() for _ in range(3 * hid)], "b_hh": [g() for _ in range(3 * hid)],
         "r_ih": [[g() for _ in range(din)] for _ in range(hid)],
         "r_hh": [[g() for _ in range(hid)] for _ in range(hid)],
         "rb_ih": [g() for _ in range(hid)], "rb_hh": [g() for _ in range(hid)],
         "tw": [f32(1 / 10 ** (j * 9 / (dt - 1))) for j in range(dt)], "tb": [g() for _ in range(dt)]}
    mails = [[g() for _ in range(mail)] for _ in range(rows)]
    h = [[g() for _ in range(hid)] for _ in range(rows)]
    ts = [f32(rng.random() * 1e4) for _ in range(rows)]
    mem_ts = [f32(rng.random() * 1e3) for _ in range(rows)]
    gru, rnn = [], []
    for i in range(rows):
        t = f32(ts[i] - mem_ts[i])
        x = mails[i] + [math.cos(f32(f32(t * P["tw"][j]) + P["tb"][j])) for j in range(dt)]
        gi = linear(x, P["w_ih"], P["b_ih"])
        gh = linear(h[i], P["w_hh"], P["b_hh"])
        r = [sigmoid(gi[j] + gh[j]) for j in range(hid)]
        z = [sigmoid(gi[hid + j] + gh[hid + j]) for j in range(hid)]
        nn = [math.tanh(gi[2 * hid + j] + r[j] * gh[2 * hid + j]) for j in range(hid)]
        gru.append([(1 - z[j]) * nn[j] + z[j] * h[i][j] for j in range(hid)])
        ri = linear(x, P["r_ih"], P["rb_ih"])
        rh = linear(h[i], P["r_hh"], P["rb_hh"])
        rnn.append([math.tanh(ri[j] + rh[j]) for j in range(hid)])
    return {"P": P, "mails": mails, "h": h, "ts": ts, "mem_ts": mem_ts, "gru": gru, "rnn": rnn}


def main():
    rng = random.Random(20240611)
    fixtures = {
        "bookkeeping.json": bookkeeping(rng),
        "softmax.json": softmax_cases(rng),
        "aggregation.json": aggregation_cases(rng),
        "fused_attn.json": fused_attn_case(rng),
        "tgat_layer_tiny.json": tgat_case(rng),
        "time_weight.json": time_weight(),
        "mfg.json": mfg_case(),
        "memory.json": memory_case(),
        "recurrent.json": recurrent_case(),
    }
    for name, data in fixtures.items():
        with open(os.path.join(HERE, name), "w") as fh:
            json.dump(data, fh, separators=(",", ":"))
    print("wrote", ", ".join(fixtures))


if __name__ == "__main__":
    main()
