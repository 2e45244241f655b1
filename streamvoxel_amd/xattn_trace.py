"""Wave timelines of the cross-attention kernel (a diagnostic, not part of the product path).

    python -m streamvoxel_amd.build --trace          # once, on the build host: libsvhip_trace.so
    python -m streamvoxel_amd.xattn_trace [--raw out.npy]
    python -m streamvoxel_amd.xattn_trace --balance   # product library: equal vs the workload's window lengths
    python -m streamvoxel_amd.xattn_trace --sequence [--lib path/libsvhip.so]   # 12 layers back to back

Runs one layer of the 8-window step workload (12 x 64 heads, 1024 queries, L_b = 1552 + 1024 k_b keys, bf16 cache,
V stored transposed) through the instrumented build of `xattn_fwd_kernel` (csrc/xattn.hip, -DSVHIP_XATTN_TRACE) and
prints a summary of what the waves did:

* per 32-key half, the median time (s_memtime ticks) of its phases: score product (operand reads, four 32x32x16
  products, until the scores are read back), exponentials and packs (VALU), row-sum readback (two 16x16x32 products
  and the wait for them), second product issue; and the wait at the block's barrier;
* per SIMD (HW_ID / XCC_ID of the three resident waves), the share of time in which one wave is in its VALU phase
  while another is in a product phase, only product phases run, only VALU phases run;
* per CU, how many waves per SIMD stay resident across the CU's span (the tail as short windows finish);
* the duration of the waves by window length.

s_memtime is a per-CU counter, so stamps are only compared within one CU. The instrumentation itself slows the
kernel (the stamps order the instructions around them); the launch time is printed next to the product kernel's.
"""
from __future__ import annotations

import argparse
import collections
import ctypes
import math
import os
import sys

import numpy as np
import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.build import TRACE_LIB

BLOCK0, BLOCKS, WORDS = 4, 8, 4 + 8 * 11          # the kernel's kTraceBlock0, kTraceBlocks, kTraceWords
WINDOWS, HEADS, HEAD_DIM, QUERIES = 8, 12, 64, 1024
LENGTHS = [7696, 1552, 6672, 4624, 4624, 9744, 4624, 8720]   # the step workload's key counts (seed 2026)


def run(seed=0):
    """One traced launch; returns (raw trace [waves, WORDS] int64, traced launch us, product launch us)."""
    if not os.path.exists(TRACE_LIB):
        raise RuntimeError(f'{TRACE_LIB} is not built; run `python -m streamvoxel_amd.build --trace` first')
    _lib.LIB_PATH = TRACE_LIB
    lib = _lib.load()
    lib.svhip_xattn_trace_set.argtypes = [ctypes.c_void_p]
    lib.svhip_xattn_trace_set.restype = ctypes.c_int
    from streamvoxel_amd.stream.attention import attention
    dev = torch.device('cuda:0')
    g = torch.Generator(device=dev).manual_seed(seed)
    kcap = max(LENGTHS) + (-max(LENGTHS)) % 64
    k = (torch.randn(WINDOWS, HEADS, kcap, HEAD_DIM, device=dev, generator=g) / 8).bfloat16()
    vt = (torch.randn(WINDOWS, HEADS, HEAD_DIM, kcap, device=dev, generator=g) / 8).bfloat16()
    q = (torch.randn(WINDOWS, QUERIES, HEADS, HEAD_DIM, device=dev, generator=g) / 8).bfloat16().transpose(1, 2)
    lengths = torch.tensor(LENGTHS, dtype=torch.int32, device=dev)
    out = torch.empty(WINDOWS, QUERIES, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev).transpose(1, 2)

    def launch():
        attention(q, k, vt.transpose(2, 3), lengths=lengths, out=out)

    def timed():
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        launch()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) * 1e3

    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    plain_us = min(timed() for _ in range(5))
    grid = WINDOWS * HEADS * math.ceil(QUERIES / 128)
    buf = torch.zeros(grid * 4 * WORDS, dtype=torch.int64, device=dev)
    if lib.svhip_xattn_trace_set(ctypes.c_void_p(buf.data_ptr())) != 0:
        raise RuntimeError('svhip_xattn_trace_set failed')
    traced_us = timed()
    if lib.svhip_xattn_trace_set(None) != 0:
        raise RuntimeError('svhip_xattn_trace_set failed')
    return buf.cpu().numpy().reshape(-1, WORDS), traced_us, plain_us


def balance(seed=0, reps=20, replays=5):
    """The product kernel on the workload's window lengths and on equal lengths with (almost) the same total keys
    (every window at the mean rounded down to 64): microseconds per launch from HIP events around graph replays of
    `reps` back-to-back launches. Tells how much the unequal windows (the tail) cost."""
    from streamvoxel_amd.stream.attention import attention
    dev = torch.device('cuda:0')
    _lib.load()
    g = torch.Generator(device=dev).manual_seed(seed)
    kcap = max(LENGTHS) + (-max(LENGTHS)) % 64
    k = (torch.randn(WINDOWS, HEADS, kcap, HEAD_DIM, device=dev, generator=g) / 8).bfloat16()
    vt = (torch.randn(WINDOWS, HEADS, HEAD_DIM, kcap, device=dev, generator=g) / 8).bfloat16()
    q = (torch.randn(WINDOWS, QUERIES, HEADS, HEAD_DIM, device=dev, generator=g) / 8).bfloat16().transpose(1, 2)
    out = torch.empty(WINDOWS, QUERIES, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev).transpose(1, 2)
    mean = sum(LENGTHS) // WINDOWS // 64 * 64
    res = {}
    for name, lens in (('warm-up', LENGTHS), ('equal', [mean] * WINDOWS), ('workload', LENGTHS),
                       ('equal_again', [mean] * WINDOWS), ('workload_again', LENGTHS)):
        lengths = torch.tensor(lens, dtype=torch.int32, device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            attention(q, k, vt.transpose(2, 3), lengths=lengths, out=out)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                attention(q, k, vt.transpose(2, 3), lengths=lengths, out=out)
        graph.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(replays):
            graph.replay()
        ev[1].record()
        torch.cuda.synchronize()
        res[name] = (ev[0].elapsed_time(ev[1]) * 1e3 / (reps * replays), sum(lens))
        del graph
    return res


def sequence(lib_path=None, layers=12, seed=0, replays=10):
    """Microseconds per launch of `layers` attention layers launched back to back in one graph, each over its own
    cache (the step's sequence of layers, every layer's K/V read from HBM), with the library at `lib_path` (default:
    the product library). An older build of the library may lack entry points added since: only the ones it
    exports are declared (the attention entry point has kept its signature)."""
    if lib_path is not None:
        _lib.LIB_PATH = os.path.abspath(lib_path)
        exported = ctypes.CDLL(_lib.LIB_PATH)
        for name in list(_lib.SIGNATURES):
            if not hasattr(exported, name):
                del _lib.SIGNATURES[name]
    _lib.load()
    from streamvoxel_amd.stream.attention import attention
    dev = torch.device('cuda:0')
    g = torch.Generator(device=dev).manual_seed(seed)
    kcap = max(LENGTHS) + (-max(LENGTHS)) % 64
    lengths = torch.tensor(LENGTHS, dtype=torch.int32, device=dev)
    caches = [((torch.randn(WINDOWS, HEADS, kcap, HEAD_DIM, device=dev, generator=g) / 8).bfloat16(),
               (torch.randn(WINDOWS, HEADS, HEAD_DIM, kcap, device=dev, generator=g) / 8).bfloat16())
              for _ in range(layers)]
    qs = [(torch.randn(WINDOWS, QUERIES, HEADS, HEAD_DIM, device=dev, generator=g) / 8).bfloat16().transpose(1, 2)
          for _ in range(layers)]
    out = torch.empty(WINDOWS, QUERIES, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev).transpose(1, 2)

    def step():
        for (k, vt), q in zip(caches, qs):
            attention(q, k, vt.transpose(2, 3), lengths=lengths, out=out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(replays):
        graph.replay()
    ev[1].record()
    torch.cuda.synchronize()
    return ev[0].elapsed_time(ev[1]) * 1e3 / (replays * layers)


def summarize(raw):
    """The summary lines of a raw trace [waves, WORDS]."""
    t = raw.astype(np.int64)
    hw = t[:, 0] & 0xffffffff
    xcc = (t[:, 0] >> 32) & 0xf
    simd = (hw >> 4) & 3
    cu = (hw >> 8) & 0xf
    sh = (hw >> 12) & 1
    se = (hw >> 13) & 7
    nfull = t[:, 1] & 0xffff
    t0, t1 = t[:, 2], t[:, 3]
    s = t[:, 4:].reshape(-1, BLOCKS, 11)   # per block: (a, s, v, r, c) for halves 0 and 1, then the barrier
    lines = [f'waves {len(t)}, SIMDs {len(set(zip(xcc, se, sh, cu, simd)))}, '
             f'resident waves per SIMD {dict(collections.Counter(collections.Counter(zip(xcc, se, sh, cu, simd)).values()))}']
    d = np.diff(s, axis=2)
    phases = [('score product (a->s)', [0, 5]), ('exponentials + packs (s->v)', [1, 6]),
              ('row-sum readback (v->r)', [2, 7]), ('second product issue (r->c)', [3, 8])]
    lines.append('per 32-key half, ticks (median / p10 / p90 over waves, sampled blocks 4-11):')
    for name, idx in phases:
        x = d[:, :, idx].ravel()
        lines.append(f'  {name:30s} {np.median(x):7.0f} {np.percentile(x, 10):7.0f} {np.percentile(x, 90):7.0f}')
    x = (s[:, :, 10] - s[:, :, 9]).ravel()
    lines.append(f'  {"after the block, to the barrier":30s} {np.median(x):7.0f} {np.percentile(x, 10):7.0f} '
                 f'{np.percentile(x, 90):7.0f}')
    x = (s[:, :, 10] - s[:, :, 0]).ravel()
    lines.append(f'  {"whole block (two halves)":30s} {np.median(x):7.0f} {np.percentile(x, 10):7.0f} '
                 f'{np.percentile(x, 90):7.0f}')
    simds = collections.defaultdict(list)
    for i in range(len(t)):
        simds[(xcc[i], se[i], sh[i], cu[i], simd[i])].append(i)
    tot = both = only_v = only_m = 0
    for ws in simds.values():
        lo = max(s[i, 0, 0] for i in ws)
        hi = min(s[i, -1, 10] for i in ws)
        if len(ws) < 2 or hi - lo < 2000:
            continue
        grid = np.arange(lo, hi, 4)
        inv = np.zeros(len(grid), int)
        inm = np.zeros(len(grid), int)
        for i in ws:
            for r in s[i]:
                for a0, a1, valu in ((r[0], r[1], 0), (r[1], r[2], 1), (r[2], r[4], 0), (r[5], r[6], 0),
                                     (r[6], r[7], 1), (r[7], r[9], 0)):
                    sel = (grid >= a0) & (grid < a1)
                    (inv if valu else inm)[sel] += 1
        tot += len(grid)
        both += int(((inv > 0) & (inm > 0)).sum())
        only_v += int(((inv > 0) & (inm == 0)).sum())
        only_m += int(((inv == 0) & (inm > 0)).sum())
    lines.append(f'per SIMD over the sampled blocks of its three waves: one wave in its VALU phase while another is '
                 f'in a product phase {both / tot:.3f}; only product phases {only_m / tot:.3f}; only VALU phases '
                 f'{only_v / tot:.3f}; neither {1 - (both + only_m + only_v) / tot:.3f}')
    cus = collections.defaultdict(list)
    for i in range(len(t)):
        cus[(xcc[i], se[i], sh[i], cu[i])].append(i)
    occ, mean = [], []
    for ws in cus.values():
        ws = np.array(ws)
        base, end = t0[ws].min(), t1[ws].max()
        g = np.linspace(base, end, 20, endpoint=False) + (end - base) / 40
        occ.append([np.sum((t0[ws] <= v) & (t1[ws] > v)) / 4 for v in g])
        mean.append((t1[ws] - t0[ws]).sum() / 4 / (end - base))
    lines.append('waves per SIMD across each CU\'s span (20 steps, mean over CUs): '
                 + ' '.join(f'{a:.2f}' for a in np.mean(occ, axis=0)) + f'; time average {np.mean(mean):.2f}')
    lines.append('wave durations by window length (ticks, median):')
    for n in sorted(set(nfull.tolist())):
        sel = nfull == n
        lines.append(f'  {n:4d} full blocks: {np.median(t1[sel] - t0[sel]):9.0f} ({np.median(t1[sel] - t0[sel]) / n:6.0f} '
                     f'per block), {int(sel.sum())} waves')
    return lines


def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument('--raw', help='also save the raw trace (.npy)')
    p.add_argument('--balance', action='store_true',
                   help='time the product kernel on the workload\'s lengths and on equal lengths instead of tracing')
    p.add_argument('--sequence', action='store_true',
                   help='time 12 layers launched back to back, each over its own cache (no tracing)')
    p.add_argument('--lib', help='with --sequence: the library to time (default: the product library)')
    args = p.parse_args(argv)
    if args.sequence:
        us = sequence(args.lib)
        print(f'{args.lib or _lib.LIB_PATH}: {us:.2f} us per layer in a sequence of 12', flush=True)
        return 0
    if args.balance:
        for name, (us, keys) in balance().items():
            if name == 'warm-up':
                continue
            print(f'{name:15s} {us:7.1f} us per launch ({keys} keys)', flush=True)
        return 0
    raw, traced_us, plain_us = run()
    if args.raw:
        np.save(args.raw, raw)
    print(f'product kernel {plain_us:.1f} us per launch; instrumented launch {traced_us:.1f} us', flush=True)
    for line in summarize(raw):
        print(line, flush=True)


if __name__ == '__main__':
    sys.exit(main())
