"""Sampler output -> device blocks (utils.py:67-87 `to_dgl_blocks`), built for the fused path.

The reference builds a DGL block per sampler result on the host and moves it with pageable
copies. Here every array of one result (row, col, node ids, dt, ts, edge ids) is packed
into one pinned staging buffer and crosses PCIe in one asynchronous copy on the current
stream; the blocks' views of it are cast on the device, and the destination offsets are
derived there when a layer first asks for them (`Block.rowptr`). Staging buffers are reused
only after the copy that last read them has completed (an event per buffer).

A sampler result is any object with the accessors of the FAST sampler's results
(sampler_core.cpp): row(), col() (int32 [E]), nodes() (int64 [dim_in]), dts(), ts()
(float32 [dim_in]), eid() (int64 [E]), dim_in(), dim_out().
"""
from __future__ import annotations

from typing import List, Optional

import numpy as np
import torch

from .tgat import Block

_ALIGN = 16


class PinnedStager:
    """Reusable pinned host buffers for H2D transfers, used round-robin; a buffer is
    refilled only after the copy that last read it has finished."""

    def __init__(self, buffers: int = 2):
        self._bufs: List[Optional[torch.Tensor]] = [None] * buffers
        self._events: List[Optional[torch.cuda.Event]] = [None] * buffers
        self._next = 0

    def transfer(self, arrays: List[np.ndarray], device) -> List[torch.Tensor]:
        """Device tensors equal to ``arrays`` (one packed asynchronous copy)."""
        offs, total = [], 0
        for a in arrays:
            offs.append(total)
            total += -(-a.nbytes // _ALIGN) * _ALIGN
        i = self._next
        self._next = (i + 1) % len(self._bufs)
        if self._events[i] is not None:
            self._events[i].synchronize()
        buf = self._bufs[i]
        if buf is None or buf.numel() < total:
            buf = torch.empty(max(total, 1), dtype=torch.uint8, pin_memory=True)
            self._bufs[i] = buf
        host = buf.numpy()
        for a, o in zip(arrays, offs):
            host[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        dev = torch.empty(max(total, 1), dtype=torch.uint8, device=device)
        dev[:total].copy_(buf[:total], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._events[i] = ev
        out = []
        for a, o in zip(arrays, offs):
            t = dev[o:o + a.nbytes].view(_torch_dtype(a.dtype))
            out.append(t.view(a.shape))
        return out


def _torch_dtype(dt: np.dtype) -> torch.dtype:
    return {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64,
            np.dtype(np.float32): torch.float32, np.dtype(np.float64): torch.float64}[np.dtype(dt)]


def _block(row, col, nodes, dts, ts, eid, dim_in: int, dim_out: int, reverse: bool) -> Block:
    if not reverse:   # edges col -> row: sources dim_in, destinations dim_out
        src, dst, n_src, n_dst = col.long(), row.long(), dim_in, dim_out
    else:
        src, dst, n_src, n_dst = row.long(), col.long(), dim_out, dim_in
    b = Block(src, dst, n_src, n_dst)
    data = b.srcdata if not reverse else b.dstdata
    data["ID"] = nodes
    data["ts"] = ts
    skip = n_dst if not reverse else n_src
    b.edata["dt"] = dts[skip:]
    b.edata["ID"] = eid
    return b


def to_blocks(ret, hist: int = 1, reverse: bool = False, device="cuda:0",
              stager: Optional[PinnedStager] = None) -> List[List[Block]]:
    """utils.py:67-87: one block per sampler result, grouped ``hist`` at a time, the groups
    reversed (bottom layer first). On a GPU device the arrays travel through ``stager``
    (pinned, asynchronous, one copy per result); on the CPU they are wrapped as they are."""
    device = torch.device(device)
    blocks = []
    for r in ret:
        arrays = [np.asarray(r.row()), np.asarray(r.col()), np.asarray(r.nodes()),
                  np.asarray(r.dts()), np.asarray(r.ts()), np.asarray(r.eid())]
        if device.type == "cuda":
            stager = stager if stager is not None else PinnedStager()
            t = stager.transfer(arrays, device)
        else:
            t = [torch.from_numpy(np.ascontiguousarray(a)) for a in arrays]
        blocks.append(_block(*t, int(r.dim_in()), int(r.dim_out()), reverse))
    groups = list(map(list, zip(*[iter(blocks)] * hist)))
    groups.reverse()
    return groups
