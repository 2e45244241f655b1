"""Benchmark of the per-step generation hot path on one MI355X.

Workload (one "step" = one HIP-graph replay): 8 windows (slots) of [256,16,16] voxels, 12 cross-attention layers
(bf16, 12 heads x 64, 1024 queries per window, cached K/V of L_b = 1552 + 1024 k_b keys, k_b ~ U{0..8}) followed by
the EASE selection of the step over [8 x 65536, 256] fp32 logits (entropy, 4^3 block quota with trim / top-up,
commit of the chosen voxels). A window is 26 forwards: one low-entropy-last marking step and 25 solid steps with
the quarter-cosine quotas; the high-entropy share of the logits drifts from 30% to 5% over the window.

  value = voxels/s = 8 * 65536 / (26 * t_step)

The backbone (self-attention, MLP), the logit producer and the categorical sampling tail are not part of the step.
Queries are drawn N(0,1)/8 per step and layer, logits per step, all resident in HBM before timing; K/V are
projected once from seeded context tokens with random-init weights (no checkpoint is published).

Prints one JSON line (rank 0). `--gpus N` with N > 1 is refused: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = 'voxels/sec on 1 GPU (8 slots); cross-attn MFMA util; EASE select HBM GB/s'
SLOTS, LAYERS, HEADS, HEAD_DIM, QUERIES, WIDTH = 8, 12, 12, 64, 1024, 768
SHAPE, CLASSES, BLOCK, STEPS_PER_WINDOW = (256, 16, 16), 256, 4, 26
VOXELS = SHAPE[0] * SHAPE[1] * SHAPE[2]
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
LAST_EPS = 1e-4


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=26)
    p.add_argument('--warmup', type=int, default=26)
    p.add_argument('--seed', type=int, default=2026)
    p.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    p.add_argument('--cpu-seconds', type=float, default=12.0, help='bounded CPU sample budget')
    p.add_argument('--kv-dtype', default='bf16', choices=['bf16', 'fp8'])
    p.add_argument('--no-forward', action='store_true', help='skip the whole-step forward component')
    p.add_argument('--forward-only', action='store_true',
                   help='time only the whole-step forward (shipped shape) and print its line')
    p.add_argument('--no-c5', action='store_true', help='skip the 64-slot e4m3 stress component')
    p.add_argument('--kernel', choices=['xattn', 'xattn_e4m3', 'xattn_layouts', 'select', 'select_planes',
                                        'select_c304', 'c5_xattn', 'c5', 'gemm_bf16'],
                   help='build only that kernel\'s inputs (the step\'s layer-0 attention or its first solid '
                        'selection), time 20 back-to-back launches and print one line: the run to profile')
    return p.parse_args()


def window_schedule(last_counts):
    """Per window slot: the 25 solid quotas of a quarter-cosine schedule with the deferred count taken from the
    tail (the smallest cap giving 25 positive quotas)."""
    from streamvoxel_amd.sampling.low_entropy_last import low_entropy_last_quotas
    out = []
    for n_last in last_counts:
        cap = STEPS_PER_WINDOW - 1
        while True:
            q = low_entropy_last_quotas(VOXELS, cap, n_last)
            if len(q) >= STEPS_PER_WINDOW - 1:
                break
            cap += 1
        out.append(q[:STEPS_PER_WINDOW - 1] if len(q) == STEPS_PER_WINDOW - 1 else q)
    return out


class Workload:
    def __init__(self, dev, seed, kv_dtype):
        import torch
        from streamvoxel_amd import synth
        from streamvoxel_amd.stream.step import CachedContext, EaseSelect

        self.dev = dev
        g = torch.Generator(device=dev).manual_seed(seed)
        self.lengths = synth.kv_lengths(SLOTS, seed)
        kv_cap = max(self.lengths)
        log(f'kv lengths {self.lengths}')
        self.ctx = CachedContext(LAYERS, SLOTS, HEADS, HEAD_DIM, synth.MAX_KEYS, dev, kv_dtype)
        # K/V projected once per window from seeded context tokens (random-init projection per layer).
        for layer in range(LAYERS):
            w = torch.randn(WIDTH, 2 * WIDTH, device=dev, generator=g) / math.sqrt(WIDTH)
            for b, L in enumerate(self.lengths):
                tokens = torch.randn(L, WIDTH, device=dev, generator=g)
                kv = (tokens @ w).reshape(L, 2, HEADS, HEAD_DIM).permute(1, 2, 0, 3)   # [2, H, L, D]
                self.ctx.write(layer, b, kv[0].to(torch.bfloat16), kv[1].to(torch.bfloat16))
        # Queries: one [8,12,1024,64] bf16 tensor per (step, layer), produced in the projection's [B,Q,H,D] layout.
        self.q = [[(torch.randn(SLOTS, QUERIES, HEADS, HEAD_DIM, device=dev, generator=g) / 8).to(torch.bfloat16)
                   .transpose(1, 2) for _ in range(LAYERS)] for _ in range(STEPS_PER_WINDOW)]
        self.o = [torch.empty(SLOTS, QUERIES, HEADS, HEAD_DIM, dtype=torch.bfloat16, device=dev)
                  for _ in range(LAYERS)]
        # Marking logits: certain air (class 0 + 30) above a seeded terrain height per column.
        self.sel = EaseSelect(SLOTS, SHAPE, CLASSES, BLOCK, dev, air_ids=(0,))
        mark = torch.empty(SLOTS * VOXELS, CLASSES, device=dev)
        synth.bimodal_logits_(mark, 0.7, generator=g)
        height = torch.randint(64, 192, (SLOTS, 1, SHAPE[1], SHAPE[2]), device=dev, generator=g)
        y = torch.arange(SHAPE[0], device=dev).reshape(1, -1, 1, 1)
        air = (y > height).reshape(-1)
        mark[air, 0] += 30.0
        self.mark_logits = mark
        # Solid-step logits, the uncertain share drifting 30% -> 5%.
        solid = STEPS_PER_WINDOW - 1
        self.logits = []
        for s in range(solid):
            x = torch.empty(SLOTS * VOXELS, CLASSES, device=dev)
            synth.bimodal_logits_(x, 1.0 - synth.high_entropy_share(s, solid), generator=g)
            self.logits.append(x)
        # One marking pass (eager) gives the deferred counts -> per-slot quotas (host, once per window).
        self.sel.tokens.fill_(CLASSES)
        self.sel.last.zero_()
        self.sel.mark(self.mark_logits, LAST_EPS)
        torch.cuda.synchronize()
        self.last_counts = self.sel.last.sum(1).tolist()
        self.quotas = window_schedule(self.last_counts)
        log(f'last counts {self.last_counts}; solid quotas slot0 {self.quotas[0][:4]}...{self.quotas[0][-2:]}')
        orders = [torch.randperm(VOXELS // BLOCK ** 3, generator=torch.Generator().manual_seed(seed + 9173 + b))
                  for b in range(SLOTS)]
        for b in range(SLOTS):
            self.sel.bind_window(b, orders[b])
        # Per-step scalar tables (copied into the select buffers inside each step's graph).
        ks, coms, fracs = [], [], []
        for s in range(solid):
            k = [self.quotas[b][s] for b in range(SLOTS)]
            com = [sum(self.quotas[b][:s]) for b in range(SLOTS)]
            fr = [(com[b] + k[b]) / (VOXELS - self.last_counts[b]) for b in range(SLOTS)]
            ks.append(torch.tensor(k, dtype=torch.int64, device=dev))
            coms.append(torch.tensor(com, dtype=torch.int64, device=dev))
            fracs.append(torch.tensor(fr, dtype=torch.float64, device=dev))
        self.k_tab, self.com_tab, self.frac_tab = ks, coms, fracs
        self.bad_seen = torch.zeros(SLOTS, dtype=torch.bool, device=dev)
        self.flops_per_layer = 4 * HEADS * HEAD_DIM * QUERIES * sum(self.lengths)
        self.select_bytes = SLOTS * VOXELS * (CLASSES * 4 + 8 + 1 + 1)

    # -- step bodies (captured)
    def attention_layers(self, step):
        for layer in range(LAYERS):
            self.ctx.attend(layer, self.q[step][layer], out=self.o[layer].transpose(1, 2))

    def selection(self, step):
        """Everything of a step but the attention layers: step 0 marks, step 1 + s is solid step s."""
        if step == 0:
            self.sel.tokens.fill_(CLASSES)
            self.sel.last.zero_()
            self.sel.mark(self.mark_logits, LAST_EPS)
            return
        s = step - 1
        self.sel.run(self.logits[s], scalars=(self.k_tab[s], self.com_tab[s], self.frac_tab[s]))
        self.bad_seen |= self.sel.bad
        self.sel.tokens.masked_fill_(self.sel.chosen.view(SLOTS, VOXELS), 1)
        if s == STEPS_PER_WINDOW - 2:
            self.sel.tokens.masked_fill_(self.sel.last, 0)     # finish: deferred voxels become air

    def step(self, step):
        self.attention_layers(step)
        self.selection(step)

    def _graphs(self, body):
        from streamvoxel_amd.stream.engine import StepGraphs
        graphs = StepGraphs(self.dev, body, range(STEPS_PER_WINDOW), warmup=1)
        if not graphs.ok:
            raise RuntimeError('the step graphs could not be captured')
        self.bad_seen.zero_()
        return [graphs.graphs[step].replay for step in range(STEPS_PER_WINDOW)]

    def capture(self):
        """One HIP graph per step of the window (the marking step, then the 25 solid steps), captured by the
        engine's `StepGraphs`; returns the callables that replay them."""
        return self._graphs(self.step)

    def capture_split(self):
        """The same steps as two graphs each, the attention layers and the rest, so that HIP events between them
        time the layers inside the step sequence; returns (layers, rest) lists of replay callables."""
        return self._graphs(self.attention_layers), self._graphs(self.selection)


def time_events(fn, reps, warm=3):
    import torch
    for _ in range(warm):
        fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps / 1e3   # seconds per call


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None where it is not readable."""
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return None


def time_graph(fn, reps, replays=5):
    """Seconds per call of `fn` from HIP events around replays of one graph of `reps` back-to-back calls (no host
    gaps between the launches), recorded on the stream the graph launches on."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / (reps * replays) / 1e3


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (a line
    `traffic <kernel> <bytes>`), or None when there is none."""
    path = os.path.join(ROOT, 'profiles', 'hbm_traffic_8slot.md')
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.strip().strip('`').split()
            if len(parts) == 3 and parts[0] == 'traffic' and parts[1] == kernel:
                return float(parts[2])
    return None


def measured_peaks(dev):
    import torch
    out = {}
    a = torch.empty(1 << 28, dtype=torch.float32, device=dev)     # 1 GiB
    b = torch.empty_like(a)
    a.normal_()
    t = time_events(lambda: b.copy_(a), 10)
    out['copy_GBps'] = 2 * a.numel() * 4 / t / 1e9
    del a, b
    m = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    n = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    t = time_events(lambda: torch.mm(m, n), 10)
    out['bf16_gemm_TFLOPs'] = 2 * 8192 ** 3 / t / 1e12
    return out


def cpu_baseline(w, budget_s):
    """The oracle (CPU restatement of the reference path) on the host cores, on a bounded sample: masked fp32 SDPA
    over the padded keys of one layer, the 8 windows in turn, and the entropy + block-quota selection of one window,
    four attention samples per selection, until `budget_s` of wall time is spent; extrapolated linearly to the full
    step (8 windows x 12 layers + 8 selections)."""
    import numpy as np
    import torch

    from oracle import attention as A
    from oracle import sampling as S
    threads = torch.get_num_threads()
    kcap = w.ctx.kv_cap
    lengths = torch.tensor(w.lengths, dtype=torch.int64)
    q = w.q[1][0].float().cpu()
    k = w.ctx.k[0].float().cpu()
    v = w.ctx.vt[0].float().cpu().transpose(2, 3).contiguous()
    sel_logits = w.logits[0][:VOXELS].cpu()                    # window 0, voxel-major [N, C]
    tokens = w.sel.tokens.new_full((VOXELS,), CLASSES).cpu().numpy()
    last = w.sel.last[0].cpu().numpy()
    pos = w.sel.pos[0].cpu().numpy()
    n_total = w.sel.n_total[0].cpu().numpy()
    k0 = int(w.k_tab[0][0])
    frac0 = float(w.frac_tab[0][0])
    attn_times, sel_times = [], []
    began = time.perf_counter()
    while True:
        for _ in range(4):
            b = len(attn_times) % SLOTS
            t0 = time.perf_counter()
            A.masked_sdpa(q[b:b + 1], k[b:b + 1], v[b:b + 1], lengths[b:b + 1])
            attn_times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        score = S.entropy_scores(sel_logits.T).numpy().reshape(SHAPE)
        selectable = ((tokens == CLASSES) & ~last).reshape(SHAPE)
        S.quota_select_nosync(score, selectable, k0, BLOCK, pos, frac0, n_total, 0)
        sel_times.append(time.perf_counter() - t0)
        if time.perf_counter() - began > budget_s:
            break
    t_attn = float(np.median(attn_times))          # one window, one layer
    t_sel = float(np.median(sel_times))            # one window
    t_step = SLOTS * LAYERS * t_attn + SLOTS * t_sel
    return dict(value=SLOTS * VOXELS / (STEPS_PER_WINDOW * t_step), unit='voxels/s', cores=threads, kind='port',
                sample=(f'{len(attn_times)} x masked fp32 SDPA (one window of 8 in turn, 1 layer, {HEADS}x{HEAD_DIM}, {QUERIES} '
                        f'queries, {kcap} padded keys) + {len(sel_times)} x fp32 entropy + block-quota select of one '
                        f'[256,16,16] window (C={CLASSES}); step extrapolated x{SLOTS * LAYERS} / x{SLOTS}'),
                seconds_per_step=t_step, attn_s_per_window_layer=t_attn, select_s_per_window=t_sel,
                cpu_count=os.cpu_count(), torch_threads=torch.get_num_threads(), cpu_model=cpu_model(),
                wall_s=time.perf_counter() - began)


def shipped_engine_component(dev, lengths_seed=7):
    """The shipped model's shape through the slot engine (`SlotEngine`, random weights in the reference's layout:
    the trained ones are not published): 8 slots of 256 x 16 x 16 voxels, 304 classes, 25 x 768 backbone blocks,
    13 x 384 control blocks with cross attention over a cache of 4096 prefix + 288 + 1024 k_b local keys
    (k_b ~ U{0..8}), synthetic conditions. Times (a) the captured step forward, `replay(timesteps, 8)`, with HIP
    events around back-to-back replays, and (b) one whole window of the worker's loop (stream/worker.py:378-397):
    26 forwards of `replay` + `consume_batch` over `SelectGraphs` of 8 slots (marking, 25 solid steps; the
    counter-based sampler inside the captured selection), wall time per forward including the host's one wait per
    forward and its bookkeeping."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.engine import SlotEngine
    from streamvoxel_amd.stream.slot import LowEntropyLastSlot, SelectGraphs, consume_batch
    model = synth.StepModel(seed=1)
    for p in model.parameters():
        p.data = p.data.to(torch.bfloat16)
    model = model.to(dev)
    spec = synth.WindowSpec()
    engine = SlotEngine(model, spec, dev, SLOTS, l1_cap=8, l2_cap=256)
    g = torch.Generator().manual_seed(lengths_seed)
    neighbours = torch.randint(0, 9, (SLOTS,), generator=g).tolist()
    for b, k in enumerate(neighbours):
        engine.load_slot(b, synth.condition(model, 256 * 16, 288 + 1024 * k, seed=100 + b, device=dev, scale=0.3))
    engine.wait_loads()
    lengths = engine.packed.lengths.tolist()
    engine.tokens.copy_(torch.randint(0, spec.num_classes + 1, engine.tokens.shape, device=dev,
                                      generator=torch.Generator(dev).manual_seed(3)))
    engine.replay(0.5, SLOTS)
    torch.cuda.synchronize()
    reps = 5
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        engine.replay(0.5, SLOTS)
    end.record()
    end.synchronize()
    t_forward = start.elapsed_time(end) / reps / 1e3
    slots = [LowEntropyLastSlot(engine.shape, spec.num_classes, (0,), air_token=0, last_eps=LAST_EPS, block_size=BLOCK,
                                device=dev, sampler='philox') for _ in range(SLOTS)]
    select = SelectGraphs(engine, slots)

    def window(seed0):
        for i, slot in enumerate(slots):
            slot.arm(seed0 + i, STEPS_PER_WINDOW - 1, (i, 0))
        engine.clear_tokens()
        forwards = 0
        while any(not slot.idle for slot in slots):
            count = 1 + max(i for i, slot in enumerate(slots) if not slot.idle)
            times = [slot.time() if i < count else 1.0 for i, slot in enumerate(slots)]
            consume_batch(slots, engine.replay(times, count), engine.tokens, count, select)
            forwards += 1
        return forwards

    window(0)                                   # warm: first replays of every select graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    forwards = window(1000)
    torch.cuda.synchronize()
    t_window = (time.perf_counter() - t0) / forwards
    if bool((engine.tokens == spec.num_classes).any()):
        raise RuntimeError('a window finished with uncommitted voxels')
    del engine, select, slots, model
    torch.cuda.empty_cache()
    return dict(forward_ms=t_forward * 1e3, kv_lengths=lengths, window_forwards=forwards,
                window_ms_per_forward=t_window * 1e3,
                window_voxels_per_s=SLOTS * VOXELS / (forwards * t_window))


def sampling_tail_component(w, dev, s=12):
    """The solid step's tail after the selection, for the 8 windows at solid step `s` of the schedule: the
    reference's eager form per window (nonzero_static(k) -> gather -> softmax -> torch.multinomial -> index_copy_ ->
    one D2H copy of positions and values, fast_ops.py:548-558) against the counter-based `svhip_sample_chosen`
    (one launch over the 8 windows, capturable with the selection) and its D2H copy of one int16 per voxel. Times
    with HIP events around the whole tail (the eager form includes its launch gaps)."""
    import torch
    from streamvoxel_amd.stream.sampler import sample_chosen
    w.sel.k.copy_(w.k_tab[s])
    w.sel.committed.copy_(w.com_tab[s])
    w.sel.frac.copy_(w.frac_tab[s])
    w.sel.tokens.fill_(CLASSES)
    w.sel.run(w.logits[s])
    torch.cuda.synchronize()
    ks = [int(v) for v in w.k_tab[s].tolist()]
    rows = w.logits[s].view(SLOTS, VOXELS, CLASSES)
    chosen = w.sel.chosen.view(SLOTS, VOXELS)
    tokens = w.sel.tokens.clone()
    gens = [torch.Generator(device=dev).manual_seed(b) for b in range(SLOTS)]
    hosts = [torch.empty(2 * k + 1, dtype=torch.int64, pin_memory=True) for k in ks]

    def multinomial_tail():
        for b in range(SLOTS):
            index = torch.nonzero_static(chosen[b], size=ks[b]).squeeze(1)
            probabilities = rows[b].index_select(0, index).float().softmax(-1)
            values = torch.multinomial(probabilities, 1, generator=gens[b]).squeeze(-1)
            tokens[b].index_copy_(0, index, values)
            hosts[b].copy_(torch.cat((index, values, w.sel.bad[b:b + 1].long())), non_blocking=True)

    logits5 = rows.view(SLOTS, *SHAPE, CLASSES).permute(0, 4, 1, 2, 3)
    seeds = torch.arange(SLOTS, dtype=torch.int64, device=dev)
    steps = torch.full((SLOTS,), s, dtype=torch.int64, device=dev)
    drawn = torch.empty(SLOTS, *SHAPE, dtype=torch.int16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    host16 = torch.empty(SLOTS * VOXELS, dtype=torch.int16, pin_memory=True)
    chosen5 = chosen.view(SLOTS, *SHAPE)
    tokens5 = tokens.view(SLOTS, *SHAPE)

    def philox_kernel():
        sample_chosen(logits5, chosen5, seeds, steps, drawn, err, tokens5)

    def philox_tail():
        philox_kernel()
        host16.copy_(drawn.view(-1), non_blocking=True)

    t_multi = time_events(multinomial_tail, 10)
    t_kernel = time_graph(philox_kernel, 20)
    t_philox = time_events(philox_tail, 10)
    torch.cuda.synchronize()
    assert int(err) == 0
    drawn_per_window = (drawn >= 0).view(SLOTS, -1).sum(1).tolist()
    assert drawn_per_window == ks, (drawn_per_window, ks)
    return dict(solid_step=s, k_per_window=ks, multinomial_eager_us=t_multi * 1e6,
                philox_kernel_us=t_kernel * 1e6, philox_with_d2h_us=t_philox * 1e6)


C5_SLOTS, C5_HEADS, C5_WIDTH = 64, 16, 1024


def c5_context(dev, seed, kv_dtype, p_dtype='bf16'):
    """The 64-slot quantised-context stress: one cross-attention layer's cache for 64 windows, 16 x 64 heads
    (hidden 1024), L_b = 1552 + 1024 k_b keys with k_b ~ U{0..8}, K/V projected from seeded context tokens and
    written by svhip_kv_write (e4m3 with per-(window, head) amax/448 scales, or bf16); 1024 bf16 queries per
    window in the projection's [B,Q,H,D] layout."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.step import CachedContext
    g = torch.Generator(device=dev).manual_seed(seed)
    lengths = synth.kv_lengths(C5_SLOTS, seed)
    ctx = CachedContext(1, C5_SLOTS, C5_HEADS, HEAD_DIM, synth.MAX_KEYS, dev, kv_dtype, p_dtype=p_dtype)
    w = torch.randn(C5_WIDTH, 2 * C5_WIDTH, device=dev, generator=g) / math.sqrt(C5_WIDTH)
    for b, L in enumerate(lengths):
        kv = (torch.randn(L, C5_WIDTH, device=dev, generator=g) @ w).reshape(L, 2, C5_HEADS, HEAD_DIM)
        kv = kv.permute(1, 2, 0, 3)
        ctx.write(0, b, kv[0].to(torch.bfloat16), kv[1].to(torch.bfloat16))
    q = (torch.randn(C5_SLOTS, QUERIES, C5_HEADS, HEAD_DIM, device=dev, generator=g) / 8).to(torch.bfloat16)
    return ctx, q, lengths


def c5_component(dev, seed):
    """The 64-slot quantised-context stress, timed: the cross-attention layer over the e4m3 cache in its default
    form (K/V decoded exactly to bf16 in the kernel, bf16 softmax weights: within the fp8 bar), the opt-in fp8
    second product (P rounded to e4m3, outside the bar on sharp rows), the same keys as a bf16 cache, and the EASE
    selection over [64 x 65536, 256] fp32 logits (4.3 GB). HIP events around graphs of back-to-back launches."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.step import EaseSelect
    out = {}
    for name, kv_dtype, p_dtype in (('e4m3', 'fp8', 'bf16'), ('e4m3_pfp8', 'fp8', 'e4m3'), ('bf16', 'bf16', 'bf16')):
        ctx, q, lengths = c5_context(dev, seed, kv_dtype, p_dtype)
        o = torch.empty_like(q)
        t = time_graph(lambda: ctx.attend(0, q.transpose(1, 2), out=o.transpose(1, 2)), 5)
        flops = 4 * C5_HEADS * HEAD_DIM * QUERIES * sum(lengths)
        out[f'xattn_{name}_us'] = t * 1e6
        out[f'xattn_{name}_TFLOPs'] = flops / t / 1e12
        out['flops_per_layer'] = flops
        out['kv_lengths_sum'] = sum(lengths)
        del ctx, q, o
    out['xattn_e4m3_frac_fp8_peak'] = out['xattn_e4m3_TFLOPs'] / PEAK_FP8_TFLOPS
    out['xattn_e4m3_frac_bf16_peak'] = out['xattn_e4m3_TFLOPs'] / PEAK_BF16_TFLOPS
    out['xattn_bf16_frac_bf16_peak'] = out['xattn_bf16_TFLOPs'] / PEAK_BF16_TFLOPS
    torch.cuda.empty_cache()
    g = torch.Generator(device=dev).manual_seed(seed + 5)
    sel = EaseSelect(C5_SLOTS, SHAPE, CLASSES, BLOCK, dev, air_ids=(0,))
    logits = torch.empty(C5_SLOTS * VOXELS, CLASSES, device=dev)
    synth.bimodal_logits_(logits, 0.7, generator=g)
    k = VOXELS // (STEPS_PER_WINDOW - 1)
    for b in range(C5_SLOTS):
        sel.bind_window(b, torch.randperm(VOXELS // BLOCK ** 3, generator=torch.Generator().manual_seed(b)))
        sel.set_step(b, k, 0, k / VOXELS)
    t = time_graph(lambda: sel.run(logits), 5)
    nbytes = C5_SLOTS * VOXELS * (CLASSES * 4 + 8 + 1 + 1)
    out.update(select_us=t * 1e6, select_GBps=nbytes / t / 1e9, select_frac_hbm=nbytes / t / 1e9 / PEAK_HBM_GBS,
               select_bytes=nbytes, select_bad_flag=bool(sel.bad.any()))
    del sel, logits
    torch.cuda.empty_cache()
    return out


def shipped_select(dev, quotas, reps):
    """The shipped model's selection input, the class head's bf16 rows of 304 classes (autocast) in patch order, for
    8 fresh windows with the given step quotas: (seconds per call of `EaseSelect.run`, bytes per call)."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.patches import PatchLogits
    from streamvoxel_amd.stream.step import EaseSelect
    classes = 304
    sel = EaseSelect(SLOTS, SHAPE, classes, BLOCK, dev)
    for b in range(SLOTS):
        sel.bind_window(b, torch.randperm(VOXELS // BLOCK ** 3, generator=torch.Generator().manual_seed(b)))
        sel.set_step(b, quotas[b], 0, quotas[b] / VOXELS)
    rows = synth.bimodal_logits(SLOTS * VOXELS, classes, 0.7, seed=304, device=dev).to(torch.bfloat16)
    logits = PatchLogits(rows.view(SLOTS, VOXELS // 64, 64 * classes), SHAPE, 4, classes)
    t = time_graph(lambda: sel.run(logits), reps)
    return t, SLOTS * VOXELS * (classes * 2 + 8 + 1 + 1)


def xattn_layouts(dev, seed):
    """The step's attention layer (8 windows, 12 x 64 heads, 1024 queries, the step's key lengths, bf16) over the
    K/V layouts a caller may pass: padded V^T (the cached-context layout), padded and packed (cu_seqlens) row-major
    V, packed V^T, and a prefix key mask over either padded V. Microseconds per launch (20 launches a graph) and
    whether each layout gives the bits of the padded V^T one."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.attention import attention
    g = torch.Generator(device=dev).manual_seed(seed)
    lengths = synth.kv_lengths(SLOTS, seed)
    kcap = max(lengths) + (-max(lengths)) % 64
    k = (torch.randn(SLOTS, HEADS, kcap, HEAD_DIM, device=dev, generator=g) / 8).bfloat16()
    v = (torch.randn(SLOTS, HEADS, kcap, HEAD_DIM, device=dev, generator=g) / 8).bfloat16()
    q = torch.randn(SLOTS, HEADS, QUERIES, HEAD_DIM, device=dev, generator=g).bfloat16()
    vt = v.transpose(2, 3).contiguous()                                          # [B, H, D, Kcap]
    lt = torch.tensor(lengths, dtype=torch.int32, device=dev)
    cu = torch.zeros(SLOTS + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lengths).cumsum(0)
    cu = cu.to(dev)
    kp = torch.cat([k[b, :, :L] for b, L in enumerate(lengths)], 1).contiguous()  # [H, sum L, D]
    vp = torch.cat([v[b, :, :L] for b, L in enumerate(lengths)], 1).contiguous()
    vtp = torch.cat([vt[b, :, :, :L] for b, L in enumerate(lengths)], 2).contiguous()  # [H, D, sum L]
    prefix = torch.arange(kcap, device=dev)[None] < lt[:, None]
    out = torch.empty_like(q)
    forms = {
        'padded_vt': lambda: attention(q, k, vt.transpose(2, 3), lengths=lt, out=out),
        'padded_v_rows': lambda: attention(q, k, v, lengths=lt, out=out),
        'packed_v_rows': lambda: attention(q, kp, vp, cu_seqlens=cu, out=out),
        'packed_vt': lambda: attention(q, kp, vtp.transpose(1, 2), cu_seqlens=cu, out=out),
        'key_mask_v_rows': lambda: attention(q, k, v, key_mask=prefix, out=out),
        'key_mask_vt': lambda: attention(q, k, vt.transpose(2, 3), key_mask=prefix, out=out),
    }
    flops = 4 * HEADS * HEAD_DIM * QUERIES * sum(lengths)
    res, first = {}, None
    for name, fn in forms.items():
        t = time_graph(fn, 20)
        fn()
        torch.cuda.synchronize()
        if first is None:
            first = out.clone()
        res[name] = dict(us_per_launch=t * 1e6, TFLOPs=flops / t / 1e12, same_bits=bool(torch.equal(out, first)))
    return dict(kernel='xattn_layouts', kv_lengths=lengths, flops_per_launch=flops, layouts=res)


def kernel_only(dev, args):
    """One kernel of the step alone, on the step's own inputs: the cross-attention layer (8 windows, 12 x 64 heads,
    1024 queries, the step's key lengths; bf16 or e4m3 cache) or the first solid selection (8 windows, fp32 logits
    [8 x 65536, 256] as voxel rows, or as class planes [8, 256, 65536] for `select_planes`; the shipped model's bf16
    rows of 304 classes in patch order for `select_c304`; fresh token state). 20 launches in one graph, replayed 5
    times."""
    import torch
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.step import CachedContext, EaseSelect
    if args.kernel == 'c5':
        return dict(kernel='c5', **c5_component(dev, args.seed))
    if args.kernel == 'xattn_layouts':
        return xattn_layouts(dev, args.seed)
    if args.kernel == 'gemm_bf16':           # the box's dense bf16 rate: torch.mm (hipBLASLt), 8192^3, random operands
        m = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
        n = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
        t = time_events(lambda: torch.mm(m, n), 20)
        return dict(kernel=args.kernel, us_per_launch=t * 1e6, TFLOPs=2 * 8192 ** 3 / t / 1e12,
                    flops_per_launch=2 * 8192 ** 3)
    if args.kernel == 'c5_xattn':            # the 64-slot e4m3 layer alone (for the profilers)
        ctx, q, lengths = c5_context(dev, args.seed, 'fp8')
        o = torch.empty_like(q)
        t = time_graph(lambda: ctx.attend(0, q.transpose(1, 2), out=o.transpose(1, 2)), 5)
        flops = 4 * C5_HEADS * HEAD_DIM * QUERIES * sum(lengths)
        return dict(kernel=args.kernel, us_per_launch=t * 1e6, TFLOPs=flops / t / 1e12, flops_per_launch=flops)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    lengths = synth.kv_lengths(SLOTS, args.seed)
    if args.kernel.startswith('xattn'):
        kv_dtype = 'fp8' if args.kernel == 'xattn_e4m3' else 'bf16'
        ctx = CachedContext(1, SLOTS, HEADS, HEAD_DIM, synth.MAX_KEYS, dev, kv_dtype)
        w = torch.randn(WIDTH, 2 * WIDTH, device=dev, generator=g) / math.sqrt(WIDTH)
        for b, L in enumerate(lengths):
            kv = (torch.randn(L, WIDTH, device=dev, generator=g) @ w).reshape(L, 2, HEADS, HEAD_DIM).permute(1, 2, 0, 3)
            ctx.write(0, b, kv[0].to(torch.bfloat16), kv[1].to(torch.bfloat16))
        q = (torch.randn(SLOTS, QUERIES, HEADS, HEAD_DIM, device=dev, generator=g) / 8).to(torch.bfloat16)
        o = torch.empty_like(q)
        t = time_graph(lambda: ctx.attend(0, q.transpose(1, 2), out=o.transpose(1, 2)), 20)
        flops = 4 * HEADS * HEAD_DIM * QUERIES * sum(lengths)
        return dict(kernel=args.kernel, us_per_launch=t * 1e6, TFLOPs=flops / t / 1e12, flops_per_launch=flops,
                    kv_lengths=lengths)
    if args.kernel == 'select_c304':         # the shipped model's input: bf16 rows of 304 classes in patch order
        t, nbytes = shipped_select(dev, [VOXELS // (STEPS_PER_WINDOW - 1)] * SLOTS, 20)
        return dict(kernel=args.kernel, us_per_call=t * 1e6, GBps=nbytes / t / 1e9, bytes_per_call=nbytes)
    sel = EaseSelect(SLOTS, SHAPE, CLASSES, BLOCK, dev, air_ids=(0,))
    logits = torch.empty(SLOTS * VOXELS, CLASSES, device=dev)
    synth.bimodal_logits_(logits, 0.7, generator=g)
    k = VOXELS // (STEPS_PER_WINDOW - 1)
    for b in range(SLOTS):
        sel.bind_window(b, torch.randperm(VOXELS // BLOCK ** 3, generator=torch.Generator().manual_seed(b)))
        sel.set_step(b, k, 0, k / VOXELS)
    if args.kernel == 'select_planes':       # the same logits as contiguous class planes [8, C, N]
        logits = logits.view(SLOTS, VOXELS, CLASSES).transpose(1, 2).contiguous()
    t = time_graph(lambda: sel.run(logits), 20)
    nbytes = SLOTS * VOXELS * (CLASSES * 4 + 8 + 1 + 1)
    return dict(kernel=args.kernel, us_per_call=t * 1e6, GBps=nbytes / t / 1e9, bytes_per_call=nbytes)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps(dict(error='this build measures one GPU; --gpus must be 1', n_gpus=args.gpus)), flush=True)
        sys.exit(2)
    import torch
    import streamvoxel_amd
    streamvoxel_amd.load()
    dev = torch.device('cuda:0')
    if args.forward_only:
        eng = shipped_engine_component(dev)
        print(json.dumps(dict(component='shipped_engine', slots=SLOTS, reference_fast_forward_rtx4090d_ms=44.0, **eng)),
              flush=True)
        return
    if args.kernel:
        print(json.dumps(kernel_only(dev, args)), flush=True)
        return
    t0 = time.perf_counter()
    w = Workload(dev, args.seed, args.kv_dtype)
    log(f'inputs ready in {time.perf_counter() - t0:.1f}s')
    graphs = w.capture()
    log('graphs captured')
    n_graphs = len(graphs)
    for i in range(args.warmup):
        graphs[i % n_graphs]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        graphs[i % n_graphs]()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    bad = bool(w.bad_seen.any())
    log(f'{ms_per_step:.3f} ms/step, bad={bad}')
    value = SLOTS * VOXELS / (STEPS_PER_WINDOW * ms_per_step / 1e3)

    # The attention kernel's average launch inside the step sequence: the same steps replayed as (layers, rest)
    # graph pairs, HIP events around every layers graph on the stream the graphs launch on (12 launches each; the
    # gaps between them count too).
    layer_graphs, rest_graphs = w.capture_split()
    for i in range(args.warmup):
        layer_graphs[i % n_graphs]()
        rest_graphs[i % n_graphs]()
    torch.cuda.synchronize()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.steps):
        marks[i][0].record()
        layer_graphs[i % n_graphs]()
        marks[i][1].record()
        rest_graphs[i % n_graphs]()
    torch.cuda.synchronize()
    t_layer = sum(a.elapsed_time(b) for a, b in marks) / (args.steps * LAYERS) / 1e3
    del layer_graphs, rest_graphs
    # Component timings: HIP events around graphs of back-to-back launches on the launching stream.
    t_layer_alone = time_graph(lambda: w.ctx.attend(0, w.q[1][0], out=w.o[0].transpose(1, 2)), 20)
    w.sel.k.copy_(w.k_tab[0])
    w.sel.committed.copy_(w.com_tab[0])
    w.sel.frac.copy_(w.frac_tab[0])
    w.sel.tokens.fill_(CLASSES)
    t_select = time_graph(lambda: w.sel.run(w.logits[0]), 20)
    from streamvoxel_amd.sampling.entropy import entropy_batched
    ent_out = torch.empty(SLOTS, VOXELS, device=dev)
    t_entropy = time_events(lambda: entropy_batched(w.logits[0].view(SLOTS, VOXELS, CLASSES), 'voxel_major',
                                                    out=ent_out), 20)
    from streamvoxel_amd import synth
    # The class head's own row order (patches of 4^3 voxels, stream/fast_ops.py:305-308): the same logits selected
    # in place, and the [n, C, Y, Z, X] copy the reference's forward makes before its selection.
    from streamvoxel_amd.stream.patches import PatchLogits
    patch_logits = PatchLogits(torch.empty(SLOTS, VOXELS // 64, 64 * CLASSES, device=dev), SHAPE, 4, CLASSES)
    patch_logits.rows[:, patch_logits.row_index(torch.arange(VOXELS, device=dev))] = \
        w.logits[0].view(SLOTS, VOXELS, CLASSES)
    t_select_patches = time_graph(lambda: w.sel.run(patch_logits), 20)
    t_permute = time_graph(lambda: patch_logits.class_major(), 20)
    del patch_logits
    t_select304, bytes304 = shipped_select(dev, [w.quotas[b][0] for b in range(SLOTS)], 20)
    # The same layer over an e4m3 cache (per-(window, head) scales, written by svhip_kv_write from layer 0's keys).
    from streamvoxel_amd.stream.step import CachedContext
    ctx8 = CachedContext(1, SLOTS, HEADS, HEAD_DIM, synth.MAX_KEYS, dev, kv_dtype='fp8')
    for b, L in enumerate(w.lengths):
        ctx8.write(0, b, w.ctx.k[0][b, :, :L], w.ctx.vt[0][b, :, :, :L].transpose(1, 2).contiguous())
    t_layer_e4m3 = time_graph(lambda: ctx8.attend(0, w.q[1][0], out=w.o[0].transpose(1, 2)), 20)
    del ctx8
    tail = sampling_tail_component(w, dev)
    log(f'sampling tail (8 windows, solid step {tail["solid_step"]}): multinomial eager '
        f'{tail["multinomial_eager_us"]:.1f} us, counter-based kernel {tail["philox_kernel_us"]:.1f} us '
        f'({tail["philox_with_d2h_us"]:.1f} us with its D2H copy)')
    c5 = None
    if not args.no_c5:
        c5 = c5_component(dev, args.seed)
        log(f'64-slot e4m3 stress (16x64 heads): layer {c5["xattn_e4m3_us"]:.0f} us = {c5["xattn_e4m3_TFLOPs"]:.0f} '
            f'TFLOP/s (opt-in fp8 P {c5["xattn_e4m3_pfp8_us"]:.0f} us, bf16 cache {c5["xattn_bf16_us"]:.0f} us); select '
            f'over 4.3 GB {c5["select_us"]:.0f} us = {c5["select_GBps"]:.0f} GB/s')
    eng = None
    if not args.no_forward:
        eng = shipped_engine_component(dev)
        log(f'shipped model through the slot engine (8 slots): step forward {eng["forward_ms"]:.2f} ms; worker loop '
            f'{eng["window_ms_per_forward"]:.2f} ms per forward = {eng["window_voxels_per_s"]:.0f} voxels/s')
    xattn_tflops = w.flops_per_layer / t_layer / 1e12
    select_gbs = w.select_bytes / t_select / 1e9
    entropy_bytes = SLOTS * VOXELS * (CLASSES * 4 + 4)
    peaks = measured_peaks(dev)
    log(f'xattn {t_layer * 1e6:.1f} us/layer = {xattn_tflops:.1f} TFLOP/s (e4m3 cache {t_layer_e4m3 * 1e6:.1f} us); '
        f'select {t_select * 1e6:.1f} us = '
        f'{select_gbs:.0f} GB/s; entropy {t_entropy * 1e6:.1f} us; select from the head\'s patch order '
        f'{t_select_patches * 1e6:.1f} us (the permute it avoids: {t_permute * 1e6:.1f} us); shipped bf16 C=304 '
        f'{t_select304 * 1e6:.1f} us; peaks {peaks}')
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, args.cpu_seconds)
        log(f'cpu baseline {cpu["value"]:.1f} voxels/s ({cpu["seconds_per_step"]:.2f} s/step)')
    result = dict(
        metric=METRIC, value=value, unit='voxels/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=ms_per_step, higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
        data='synthetic',
        config=dict(workload=('8-slot step: 12 cross-attn layers (bf16 MFMA, 12x64 heads, 1024 queries, cached K/V '
                              'L_b=1552+1024k_b) + EASE select over [8x65536,256] fp32 logits, one HIP graph per step; '
                              '26 steps per window'),
                    slots=SLOTS, layers=LAYERS, heads=HEADS, head_dim=HEAD_DIM, queries=QUERIES,
                    kv_lengths=w.lengths, kv_dtype=args.kv_dtype, window=list(SHAPE), classes=CLASSES, block=BLOCK,
                    steps_per_window=STEPS_PER_WINDOW, parallelism='single GPU (slots are independent)'),
        roofline=dict(kernel='xattn_fwd_kernel', bound='mfma', achieved=xattn_tflops, peak=PEAK_BF16_TFLOPS,
                      unit='TFLOP/s', frac=xattn_tflops / PEAK_BF16_TFLOPS,
                      traffic=profiled_traffic('xattn_fwd_kernel'),
                      flops_per_launch=w.flops_per_layer, avg_launch_us=t_layer * 1e6,
                      layer0_back_to_back_us=t_layer_alone * 1e6,
                      e4m3_cache_us=t_layer_e4m3 * 1e6, e4m3_cache_TFLOPs=w.flops_per_layer / t_layer_e4m3 / 1e12,
                      frac_of_box_bf16_gemm=xattn_tflops / peaks['bf16_gemm_TFLOPs']),
        roofline_select=dict(kernel='svhip_ease_select (entropy + apportion + in-block + fix)', bound='hbm',
                             achieved=select_gbs, peak=PEAK_HBM_GBS, unit='GB/s', frac=select_gbs / PEAK_HBM_GBS,
                             traffic=profiled_traffic('ease_select'), bytes_per_call=w.select_bytes,
                             avg_call_us=t_select * 1e6,
                             entropy_kernel_GBps=entropy_bytes / t_entropy / 1e9, entropy_us=t_entropy * 1e6,
                             patch_order_us=t_select_patches * 1e6,
                             patch_order_GBps=w.select_bytes / t_select_patches / 1e9,
                             shipped_bf16_c304_patch_order_us=t_select304 * 1e6,
                             shipped_bf16_c304_GBps=bytes304 / t_select304 / 1e9,
                             frac_of_box_copy=select_gbs / peaks['copy_GBps']),
        components=dict(xattn_ms_per_step=LAYERS * t_layer * 1e3, select_ms_per_step=t_select * 1e3,
                        select_from_patch_order_ms_per_step=t_select_patches * 1e3,
                        class_major_permute_ms_avoided=t_permute * 1e3,
                        selection_bad_flag_seen=bad,
                        shipped_engine=eng,
                        shipped_step_forward_plus_select_ms=(None if eng is None else
                                                             eng['forward_ms'] + t_select304 * 1e3),
                        reference_fast_forward_rtx4090d_ms=44.0,
                        sampling_tail=tail,
                        c5_64slot_e4m3=c5),
        measured_peaks=peaks,
        cpu_baseline=cpu,
    )
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
