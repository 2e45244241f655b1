"""Low-entropy-last window slots on the HIP selection kernels.

Reference counterparts: `ForwardBudget` and `LowEntropyLastSlot` (streamvoxel/stream/slot.py:12-176),
`FastLowEntropyLastSlot`, `SelectGraphs` and `consume_batch` (streamvoxel/stream/fast_ops.py:481-642). The
constructors, methods, phases, host records and random streams are the reference's: the block order is
`randperm(blocks)` on a generator seeded `seed + 9173`, and the only draws on the sample generator are the
categorical samples of the solid steps, one per chosen voxel in ascending flat (YZX) order. A trajectory therefore
equals the reference's on the same device and torch build whenever the selection masks are equal.

The device work of a window:
  * marking forward: `svhip_air_prob` and `svhip_lel_update` (column mode) into the deferred mask, one host read
    of its count (the reference's `int(last.sum())`, stream/slot.py:130);
  * solid forward: `svhip_ease_select` (entropy, selectable = unfilled & not deferred, block-quota selection, the
    `bad` flag) into static buffers, capturable in a graph; then the eager tail the reference keeps in torch
    (`nonzero_static` -> softmax -> multinomial -> `index_copy_`, fast_ops.py:548-553) and one pinned D2H copy.
    With `sampler='philox'` the tail is `svhip_sample_chosen` instead, a counter-based draw per chosen voxel inside
    the captured selection (a different random stream from the reference's), and the D2H copy is one int16 per
    voxel;
  * finish: the deferred voxels are written as `air_token`.
"""
from __future__ import annotations

from collections.abc import Mapping

import numpy as np
import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.sampling.block_quota import QuotaWorkspace, block_view
from streamvoxel_amd.sampling.low_entropy_last import low_entropy_last_quotas
from streamvoxel_amd.sampling.schedule import actual_time
from streamvoxel_amd.stream.patches import PatchLogits
from streamvoxel_amd.stream.sampler import sample_chosen
from streamvoxel_amd.stream.step import EaseSelect

ORDER_SEED_OFFSET = 9173
ENTROPY_NAMES = ('torch', 'triton', 'hip')
SAMPLERS = ('multinomial', 'philox')


def check_slot_options(entropy, sampler):
    """The slot's options, validated as the reference does (fast_ops.py:494-495): ValueError for unknown names."""
    if entropy not in ENTROPY_NAMES:
        raise ValueError(f'entropy must be one of {ENTROPY_NAMES} (each runs the HIP entropy kernel)')
    if sampler not in SAMPLERS:
        raise ValueError(f'sampler must be one of {SAMPLERS}')


class ForwardBudget:
    """Forward counting of one window (stream/slot.py:12-47): the marking forward, then one forward per solid quota.

    Kept as two counters, the window's forward total and the forwards taken so far; the phase follows from them:
    'idle' before `arm` and once every forward is taken, 'marking' before the first forward, 'solid' in between.
    `arm(total)` sets the whole-window count including the marking forward; `forward()` returns True on the forward
    that finishes the window (an idle budget takes no forward and returns False)."""

    def __init__(self):
        self.total = 0
        self.nfe = 0

    def arm(self, total):
        total = int(total)
        if total < 1:
            raise ValueError('A window needs at least the marking forward')
        self.total, self.nfe = total, 0

    @property
    def phase(self):
        if self.nfe >= self.total:
            return 'idle'
        return 'marking' if self.nfe == 0 else 'solid'

    @property
    def solid(self):
        """Solid forwards of the armed window."""
        return max(self.total - 1, 0)

    @property
    def left(self):
        """Solid forwards still to take (0 before the marking forward and once idle)."""
        return self.total - self.nfe if self.phase == 'solid' else 0

    def forward(self):
        if self.phase == 'idle':
            return False
        self.nfe += 1
        return self.nfe == self.total


def _class_major(logits, classes, total):
    """(tensor, dtype code, stride_c, stride_n) of [C, Y, Z, X] logits as the kernels read them: [C, N] with a unit
    stride along the voxels (class planes) or along the classes (a view of voxel rows). Logits that do not flatten
    so without a copy, or in another float type, are made class-major on the device."""
    if logits.dtype not in (torch.float32, torch.bfloat16):
        logits = logits.float()
    x = logits.reshape(classes, total)
    if x.stride(1) != 1 and x.stride(0) != 1:
        x = x.contiguous()
    return x, _lib.dtype_code(x.dtype), x.stride(0), x.stride(1)


class LowEntropyLastSlot:
    """One window of `shape` ([Y,Z,X]) inside a batched forward (stream/slot.py:50-176, with the solid steps of
    `FastLowEntropyLastSlot`, fast_ops.py:481-581). `entropy` takes the reference's names, 'torch' (its default)
    and 'triton' (fast_ops.py:491-496), and 'hip': each runs the HIP entropy kernel, whose scores are within 2e-6
    of float64 and so within tolerance of torch's, not bit for bit (the reference's own two are not bitwise equal
    either, fast_ops.py:421-422).
    `keep_scores=True` also leaves each solid step's fp32 scores in `self.scores` (for checking).
    `sampler` draws the chosen voxels' classes: 'multinomial' (the reference's tail: `torch.multinomial` on the
    slot's generator, eager, k-sized) or 'philox' (`svhip_sample_chosen`: a counter-based draw per voxel keyed by
    the window's seed and the solid step, inside `select` and thus inside a captured step; the host reads back one
    int16 per voxel)."""

    def __init__(self, shape, classes, air_ids, air_token, last_eps, block_size, device, entropy='torch',
                 keep_scores=False, sampler='multinomial'):
        check_slot_options(entropy, sampler)
        self.sampler = sampler
        self.shape = tuple(int(s) for s in shape)
        if len(self.shape) != 3:
            raise ValueError('shape is [Y, Z, X]')
        self.total = self.shape[0] * self.shape[1] * self.shape[2]
        self.classes = int(classes)
        self.air_ids = tuple(int(a) for a in air_ids)
        self.air_token = int(air_token)
        self.last_eps = float(last_eps)
        self.block_size = int(block_size)
        self.device = torch.device(device)
        if self.device.type != 'cuda':
            raise RuntimeError('LowEntropyLastSlot runs on the GPU; there is no CPU path')
        b = self.block_size
        if any(s % b for s in self.shape):
            raise ValueError(f'shape {self.shape} is not a multiple of block_size {b}')
        self.entropy_name = entropy
        self.phase = 'idle'
        self.target = self.seed = self.cap = None
        self.last = None
        self.quotas = None
        self.solid_calls = self.actual = self.nfe = self.last_count = 0
        self.order = self.generator = None
        self._step_map = torch.zeros(self.shape, dtype=torch.int16)
        self._values = torch.full(self.shape, -1, dtype=torch.int16)
        self._pending = None
        blocks = self.total // b ** 3
        dev = self.device
        # Static buffers at fixed addresses, so a captured `select` stays valid across windows.
        self.last_static = torch.zeros(self.shape, dtype=torch.bool, device=dev)
        self.n_total = torch.zeros(blocks, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(blocks, dtype=torch.int64, device=dev)
        self.k = torch.zeros(1, dtype=torch.int64, device=dev)
        self.committed = torch.zeros(1, dtype=torch.int64, device=dev)
        self.frac = torch.zeros(1, dtype=torch.float64, device=dev)
        self.chosen = torch.zeros(self.shape, dtype=torch.bool, device=dev)
        self.bad = torch.zeros(1, dtype=torch.bool, device=dev)
        self.scores = torch.zeros(self.shape, dtype=torch.float32, device=dev) if keep_scores else None
        self.air_index = torch.as_tensor(self.air_ids, dtype=torch.int32, device=dev)
        self.air_p = torch.zeros(self.shape, dtype=torch.float32, device=dev)
        self.workspace = QuotaWorkspace(1, self.shape, b, dev, fused=True)
        self._bound = False
        # A solid step ends on the device as `drawn` (the drawn class of every chosen voxel, -1 elsewhere), the
        # quota flag and the sampler's error flag; one copy of each to pinned host memory, then `commit_drawn`.
        self.sample_err = torch.zeros(1, dtype=torch.int32, device=dev)
        self.drawn = torch.full(self.shape, -1, dtype=torch.int16, device=dev)
        self._host16 = torch.empty(self.total, dtype=torch.int16, pin_memory=True)
        self._host_flags = torch.empty(2, dtype=torch.int32, pin_memory=True)
        if sampler == 'philox':
            self.seed_dev = torch.zeros(1, dtype=torch.int64, device=dev)
            self.step_dev = torch.zeros(1, dtype=torch.int64, device=dev)

    @property
    def idle(self):
        return self.phase == 'idle'

    @property
    def step_map(self):
        """[Y,Z,X] int16 host map: the forward that committed each voxel (0 where none yet)."""
        self._settle()
        return self._step_map

    @property
    def values(self):
        """[Y,Z,X] int16 host map: each committed voxel's class (-1 where none yet)."""
        self._settle()
        return self._values

    def _settle(self):
        """Run the host work of this slot's deferred commit, if one is waiting."""
        if self._pending is not None:
            self._pending.materialize()

    def arm(self, seed, cap, target):
        """stream/slot.py:86-103."""
        self.phase = 'marking'
        self.seed = int(seed)
        self.cap = int(cap)
        self.target = tuple(target)
        self.nfe = self.actual = self.solid_calls = self.last_count = 0
        self.quotas = None
        self.last = torch.zeros(self.shape, dtype=torch.bool, device=self.device)
        blocks = self.total // self.block_size ** 3
        order_rng = torch.Generator(device=self.device).manual_seed(self.seed + ORDER_SEED_OFFSET)
        self.order = torch.randperm(blocks, device=self.device, generator=order_rng)
        self.generator = torch.Generator(device=self.device).manual_seed(self.seed)
        if self.sampler == 'philox':
            self.seed_dev.fill_(self.seed)
            self.sample_err.zero_()
        self._settle()
        self._step_map = torch.zeros(self.shape, dtype=torch.int16)
        self._values = torch.full(self.shape, -1, dtype=torch.int16)
        self._bound = False

    def drop(self):
        self.phase = 'idle'
        self.target = None
        self.quotas = None

    def time(self, tokens=None):
        """Masked fraction mapped to model time; solid steps commit exactly their quota, so no device read."""
        if self.phase == 'idle':
            return 1.0
        committed = sum(self.quotas[:self.solid_calls]) if self.quotas else 0
        return actual_time((self.total - committed) / self.total)

    def stageable(self):
        return self.phase == 'solid' and self.quotas is not None and self.solid_calls < len(self.quotas)

    # -- marking ---------------------------------------------------------------------------------------------------

    def _mark(self, logits, tokens):
        """The marking forward (stream/slot.py:124-135): air probability, then the top run of clean voxels of every
        (z, x) column joins the deferred set."""
        lib = _lib.load()
        Y, Z, X = self.shape
        if isinstance(logits, PatchLogits):
            rows = self._patch_rows(logits)
            stream = _lib.stream_of(rows)
            _lib.check(lib.svhip_air_prob_patches(
                _lib.ptr(rows), _lib.dtype_code(rows.dtype), 1, self.classes, Y, Z, X, logits.patch, 0,
                rows.stride(0), _lib.ptr(self.air_index), int(self.air_index.numel()), _lib.ptr(self.air_p), stream),
                'svhip_air_prob_patches')
        else:
            x, code, sc, sn = _class_major(logits, self.classes, self.total)
            stream = _lib.stream_of(x)
            _lib.check(lib.svhip_air_prob(_lib.ptr(x), code, 1, self.classes, self.total, 0, sc, sn,
                                          _lib.ptr(self.air_index), int(self.air_index.numel()),
                                          _lib.ptr(self.air_p), stream), 'svhip_air_prob')
        _lib.check(lib.svhip_lel_update(_lib.ptr(self.last.view(torch.uint8)), None, _lib.ptr(self.air_p), None,
                                        self.last_eps, _lib.SVHIP_LEL_COLUMN, 1, Y, Z, X, stream),
                   'svhip_lel_update')
        self.last_count = int(self.last.sum())
        self.quotas = low_entropy_last_quotas(self.total, self.cap, self.last_count, 'quartercos')
        self.phase = 'solid'
        self.solid_calls = 0

    # -- solid steps -----------------------------------------------------------------------------------------------

    def _bind(self):
        """Once per window: the deferred mask and the block constants into the static buffers."""
        if not self._bound:
            self.last_static.copy_(self.last)
            self.n_total.copy_(block_view((~self.last).contiguous(), self.block_size).sum(1))
            self.pos[self.order] = torch.arange(len(self.order), device=self.device)
            self._bound = True

    def step_scalars(self):
        """(k, committed, frac, solid step) of the next solid step, host numbers (fast_ops.py:519-532), after the
        once-per-window binding of the static buffers."""
        self._bind()
        k = self.quotas[self.solid_calls]
        committed = sum(self.quotas[:self.solid_calls])
        return k, committed, (committed + k) / (self.total - self.last_count), self.solid_calls

    def prepare(self):
        """Per-step scalars (device fills, no H2D copy) and, once per window, the deferred mask and the block
        constants (fast_ops.py:519-532). Returns k."""
        k, committed, frac, step = self.step_scalars()
        self.k.fill_(k)
        self.committed.fill_(committed)
        self.frac.fill_(frac)
        if self.sampler == 'philox':
            self.step_dev.fill_(step)
        return k

    def _patch_rows(self, logits):
        """[N, C] rows of a one-window PatchLogits of this slot's shape and classes."""
        if len(logits) != 1 or logits.shape != self.shape or logits.classes != self.classes:
            raise ValueError(f'patch logits of {len(logits)} x {logits.shape} windows of {logits.classes} classes, '
                             f'the slot needs one {self.shape} window of {self.classes}')
        _lib.require_gpu(logits.rows)
        return logits.rows[0]

    def select(self, logits, tokens):
        """Graph-capturable (fast_ops.py:534-540): reads logits [C,Y,Z,X] (or a PatchLogits of one window: the
        class head's output in place), tokens [Y,Z,X] int64 and the static buffers; writes `chosen` and `bad` (and
        `scores` when kept). One fused kernel sequence, no host sync. With the 'philox' sampler it also draws the
        chosen voxels into `tokens` and `drawn` (the whole solid step on the device)."""
        x = self._select(logits, tokens)
        if self.sampler == 'philox':
            if not isinstance(logits, PatchLogits):
                # the class-major tensor the selection read, as [1, C, Y, Z, X] (its voxels are one strided axis)
                Y, Z, X = self.shape
                sc, sn = x.stride(0), x.stride(1)
                logits = x.as_strided((1, self.classes, Y, Z, X), (0, sc, Z * X * sn, X * sn, sn))
            sample_chosen(logits, self.chosen, self.seed_dev, self.step_dev, self.drawn, self.sample_err, tokens)

    def _select(self, logits, tokens):
        _lib.require_gpu(tokens)
        if tokens.dtype != torch.int64 or tokens.shape != self.shape or not tokens.is_contiguous():
            raise ValueError('tokens must be a contiguous int64 [Y, Z, X] buffer')
        Y, Z, X = self.shape
        lib = _lib.load()
        if isinstance(logits, PatchLogits):
            rows = self._patch_rows(logits)
            _lib.check(lib.svhip_ease_select_patches(
                _lib.ptr(rows), _lib.dtype_code(rows.dtype), self.classes, logits.patch, 0, rows.stride(0),
                _lib.ptr(tokens), self.classes, _lib.ptr(self.last_static.view(torch.uint8)), 1, Y, Z, X,
                self.block_size, _lib.ptr(self.k), _lib.ptr(self.pos), _lib.ptr(self.frac), _lib.ptr(self.n_total),
                _lib.ptr(self.committed), _lib.ptr(self.chosen.view(torch.uint8)), _lib.ptr(self.bad.view(torch.uint8)),
                _lib.ptr(self.scores), _lib.ptr(self.workspace.buffer), self.workspace.buffer.numel(),
                _lib.stream_of(rows)), 'svhip_ease_select_patches')
            return
        _lib.require_gpu(logits)
        x, code, sc, sn = _class_major(logits, self.classes, self.total)
        _lib.check(lib.svhip_ease_select(
            _lib.ptr(x), code, self.classes, self.classes * self.total, sc, sn, _lib.ptr(tokens), self.classes,
            _lib.ptr(self.last_static.view(torch.uint8)), 1, Y, Z, X, self.block_size, _lib.ptr(self.k),
            _lib.ptr(self.pos), _lib.ptr(self.frac), _lib.ptr(self.n_total), _lib.ptr(self.committed),
            _lib.ptr(self.chosen.view(torch.uint8)), _lib.ptr(self.bad.view(torch.uint8)), _lib.ptr(self.scores),
            _lib.ptr(self.workspace.buffer), self.workspace.buffer.numel(), _lib.stream_of(x)), 'svhip_ease_select')
        return x

    def stage(self, logits, tokens, graph=None):
        """Selection (eager, or a replay of `graph`, a captured `select`), then the eager tail; no host wait.
        Returns the handle `collect` takes (fast_ops.py:542-558)."""
        k = self.prepare()
        if graph is None:
            self.select(logits, tokens)
        else:
            graph.replay()
        if self.sampler == 'multinomial':
            # The reference's draw: one multinomial row per chosen voxel, in ascending voxel order, from the slot's
            # generator (the order fixes the random stream); the draws go into `drawn` like the counter-based
            # sampler's.
            index = torch.nonzero_static(self.chosen.reshape(-1), size=k).squeeze(1)
            if isinstance(logits, PatchLogits):
                rows = logits.gather(index)                                 # [k, C], voxels in index order
            else:
                rows = logits.reshape(self.classes, -1).index_select(1, index).t().contiguous()
            values = torch.multinomial(rows.float().softmax(-1), 1, generator=self.generator).squeeze(-1)
            tokens.view(-1).index_copy_(0, index, values)
            self.drawn.fill_(-1)
            self.drawn.view(-1).index_copy_(0, index, values.to(torch.int16))
        self._host16.copy_(self.drawn.view(-1), non_blocking=True)
        self._host_flags[:1].copy_(self.bad.int(), non_blocking=True)
        self._host_flags[1:].copy_(self.sample_err, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        return event, tokens

    def collect(self, staged):
        """Wait for the step's copy of the drawn classes and flags, then the host bookkeeping (`commit_drawn`)."""
        event, tokens = staged
        event.synchronize()
        if int(self._host_flags[1]):
            raise RuntimeError('probability tensor contains either `inf`, `nan` or element < 0')
        return self.commit_drawn(self._host16.numpy(), bool(self._host_flags[0]), tokens)

    def commit_drawn(self, drawn, bad, tokens, defer=False):
        """The host bookkeeping of a solid step from the drawn classes of the window (`drawn`, numpy int16 [N], -1
        where not chosen) and its quota flag: the commit's positions in ascending flat order and their values, the
        step and value maps, and the finish record after the last solid step (fast_ops.py:560-575).
        The step counters advance at once. With `defer` (and unless the step ends the window) the rest, a pass over
        the window's N drawn classes, waits in a `DeferredCommit` until it is read or `_settle` runs it; `drawn` must
        then stay unchanged until that happens."""
        if bad:
            raise AssertionError('low-entropy-last solid step did not meet its quota')
        self._settle()
        k = self.quotas[self.solid_calls]
        self.solid_calls += 1
        self.actual += 1
        self.nfe += 1
        commit = DeferredCommit(self, drawn, k, self.nfe)
        if self.solid_calls >= len(self.quotas):
            commit = commit.materialize()
            return self._finish(tokens), commit
        if not defer:
            return None, commit.materialize()
        self._pending = commit
        return None, commit

    def adopt(self, batch, index):
        """Move this slot's static device buffers into window `index` of a `PhiloxBatch` (contents kept): from then
        on they are views of the batch's window-by-window arrays, which one launch selects and samples for every
        window."""
        sel = batch.sel
        views = dict(last_static=sel.last[index].view(self.shape), n_total=sel.n_total[index],
                     pos=sel.pos[index], k=sel.k[index:index + 1], committed=sel.committed[index:index + 1],
                     frac=sel.frac[index:index + 1], chosen=sel.chosen[index].view(self.shape),
                     bad=sel.bad[index:index + 1], seed_dev=batch.seeds[index:index + 1],
                     step_dev=batch.steps[index:index + 1], drawn=batch.drawn[index], sample_err=batch.err)
        for name, view in views.items():
            view.copy_(getattr(self, name))
            setattr(self, name, view)

    def consume(self, logits, tokens):
        """One forward for this slot (stream/slot.py:117-164). `tokens` [Y,Z,X] int64 is updated in place, `logits`
        is [C,Y,Z,X] or a PatchLogits of one window. Returns (finish record or None, commit or None)."""
        if self.phase == 'idle':
            return None, None
        if self.phase == 'marking':
            self.nfe += 1
            self._mark(logits, tokens)
            if not self.quotas:
                return self._finish(tokens), None
            return None, None
        if not self.stageable():
            return self._finish(tokens), None
        return self.collect(self.stage(logits, tokens))

    def _finish(self, tokens):
        """stream/slot.py:166-176: the deferred voxels become `air_token`; the window record."""
        self._settle()
        tokens[self.last] = self.air_token
        last_cpu = self.last.cpu()
        self._step_map[last_cpu] = self.nfe
        self._values[last_cpu] = self.air_token
        record = dict(target=self.target, seed=self.seed, cap=self.cap, nfe=int(self.nfe), actual=int(self.actual),
                      last_count=int(self.last_count), last_frac=float(self.last_count) / self.total,
                      step_map=self._step_map.clone(), values=self._values.clone())
        self.phase = 'idle'
        self.target = None
        return record


# The solid steps above already run the fast (staged, capturable) path; the reference's name for that class.
FastLowEntropyLastSlot = LowEntropyLastSlot


class DeferredCommit(Mapping):
    """A solid step's commit record ({positions, values, step}, as `commit_drawn` returns it) whose host work runs
    on first read or when its slot settles: the positions of the drawn voxels in ascending flat order (a pass over
    the window's drawn classes), their values, and their entries in the slot's step and value maps. The batched
    `consume_batch` hands these out and settles them at its next call, before it overwrites the drawn classes, so
    in a worker loop that launches the next forward first that work runs while the GPU computes."""

    __slots__ = ('_slot', '_drawn', '_k', '_step', '_maps', '_data')

    def __init__(self, slot, drawn, k, step):
        self._slot, self._drawn, self._k, self._step = slot, drawn, int(k), int(step)
        self._maps = (slot._step_map, slot._values)   # this window's maps (a re-arm replaces the slot's)
        self._data = None

    def materialize(self):
        """The commit as a plain dict (computed once)."""
        if self._data is None:
            drawn = self._drawn
            positions = np.flatnonzero(drawn >= 0)
            if len(positions) != self._k:
                raise AssertionError(f'{len(positions)} voxels drawn for a quota of {self._k}')
            values = drawn[positions]
            step_map, vals = self._maps
            step_map.numpy().reshape(-1)[positions] = self._step
            vals.numpy().reshape(-1)[positions] = values
            self._data = dict(positions=positions.astype('int32'), values=values.copy(), step=self._step)
            self._drawn = None
            if self._slot._pending is self:
                self._slot._pending = None
        return self._data

    def __getitem__(self, key):
        return self.materialize()[key]

    def __iter__(self):
        return iter(self.materialize())

    def __len__(self):
        return len(self.materialize())

    def __repr__(self):
        return f'DeferredCommit({self.materialize()!r})'


class _NothingSelected:
    """Context in which every slot's quota is 0, so that a captured or warm-up `select` commits and draws nothing
    (a slot with the 'philox' sampler would otherwise draw into the engine's token rows); the quotas come back
    afterwards and the static outputs are cleared. `prepare()` sets the quota before every real step."""

    def __init__(self, slots):
        self.slots = slots

    def __enter__(self):
        self.saved = [slot.k.clone() for slot in self.slots]
        for slot in self.slots:
            slot.k.zero_()

    def __exit__(self, *exc):
        for slot, k in zip(self.slots, self.saved):
            slot.chosen.zero_()
            slot.bad.zero_()
            slot.k.copy_(k)
        return False


class PhiloxBatch:
    """Device state of the solid steps of a batch of 'philox' slots, laid out window by window at fixed
    addresses, so that one selection launch (`EaseSelect.run`: entropy, block quota, trim / top-up, `bad`) and one
    sampling launch (`svhip_sample_chosen`) serve every window of a bucket. The slots' own static buffers become
    views of it (`LowEntropyLastSlot.adopt`), so their eager paths keep working. The per-step scalars of all
    windows (k, committed, frac, solid step) sit in one device array that one host-to-device copy fills; windows
    that take no solid step in a forward get k = 0 and select and draw nothing."""

    def __init__(self, slots, tokens):
        batch = len(tokens)
        s0 = slots[0]
        self.batch, self.shape, self.total = batch, s0.shape, s0.total
        dev = s0.device
        self.sel = EaseSelect(batch, s0.shape, s0.classes, s0.block_size, dev)
        self.sel.tokens = tokens.view(batch, -1)
        self.scal = torch.zeros(4 * batch, dtype=torch.int64, device=dev)
        self.sel.k, self.sel.committed = self.scal[:batch], self.scal[batch:2 * batch]
        self.sel.frac = self.scal[2 * batch:3 * batch].view(torch.float64)
        self.steps = self.scal[3 * batch:]
        self.seeds = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.drawn = torch.full((batch, *s0.shape), -1, dtype=torch.int16, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        self.host_scal = torch.zeros(4 * batch, dtype=torch.int64, pin_memory=True)
        self.host_drawn = torch.empty((batch, s0.total), dtype=torch.int16, pin_memory=True)
        self.host_bad = torch.empty(batch, dtype=torch.uint8, pin_memory=True)
        self.host_err = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self.pending = []       # DeferredCommits over rows of host_drawn, settled before the next copy into it
        for i, slot in enumerate(slots[:batch]):
            slot.adopt(self, i)

    @staticmethod
    def fits(slots, tokens):
        """Whether `slots` can share one batch over the token rows `tokens` [batch, Y, Z, X]."""
        batch = len(tokens)
        if len(slots) < batch or batch < 1:
            return False
        s0 = slots[0]
        return all(isinstance(s, LowEntropyLastSlot) and s.sampler == 'philox' and s.shape == s0.shape
                   and s.classes == s0.classes and s.block_size == s0.block_size and s.device == s0.device
                   for s in slots[:batch]) and tuple(tokens.shape[1:]) == s0.shape

    def run(self, logits, size):
        """Selection and sampling of the first `size` windows (capturable): `logits` is a bucket's output, a
        PatchLogits or class-major [size, C, Y, Z, X]."""
        self.sel.run(logits, n=size)
        sample_chosen(logits, self.sel.chosen[:size].view(size, *self.shape), self.seeds[:size], self.steps[:size],
                      self.drawn[:size], self.err, self.sel.tokens[:size].view(size, *self.shape))


class SelectGraphs:
    """One captured `select` per (bucket, slot) over an engine's static outputs and token rows
    (fast_ops.py:584-623). `engine` provides `device`, `graphs` (non-empty once captured), `outputs`
    ({bucket size: logits [size, C, Y, Z, X] or PatchLogits}) and `tokens` ([slots, Y, Z, X] int64). The graphs are
    made by the engine's own `StepGraphs` (warm-up on a side stream, one pool, the buckets in ascending order); if
    a capture fails the dictionary stays empty and every step selects eagerly. `lookup(logits)` returns the bucket
    whose output tensor `logits` is, or None (eager logits then select eagerly)."""

    def __init__(self, engine, slots):
        from streamvoxel_amd.stream.engine import StepGraphs
        self.engine, self.slots = engine, slots
        self.graphs = {}
        self._buckets = {}
        self.batch = None
        if not getattr(engine, 'graphs', None):
            return
        outputs = engine.outputs
        self._buckets = {(out.data_ptr(), len(out)): size for size, out in outputs.items()}
        if PhiloxBatch.fits(slots, engine.tokens):
            # 'philox' slots: one graph per bucket selects and samples all its windows.
            batch = PhiloxBatch(slots, engine.tokens)
            keys = sorted(outputs)

            def body(size):
                batch.run(outputs[size], size)
        else:
            batch = None
            keys = [(size, i) for size in sorted(outputs) for i in range(size)]

            def body(key):
                size, i = key
                slots[i].select(outputs[size][i], engine.tokens[i])

        with _NothingSelected(slots[:len(engine.tokens)]), torch.inference_mode():
            captured = StepGraphs(engine.device, body, keys, warmup=1)
            torch.cuda.synchronize(engine.device)
        self.graphs = captured.graphs
        self.batch = batch if self.graphs else None

    def lookup(self, logits):
        return self._buckets.get((logits.data_ptr(), len(logits)))


def consume_batch(slots, logits, tokens, count, graphs=None):
    """`[slot.consume(logits[i], tokens[i]) for i < count]` with every staged solid step enqueued before the first
    host wait (fast_ops.py:626-642): the device work of all the batch's solid steps is queued first (each slot's
    captured select when `logits` is a bucket's output), then the host collects the slots in order. Marking and
    finishing forwards go through `consume`. Returns {index: (finished, commit)} for the non-idle slots."""
    bucket = graphs.lookup(logits) if graphs is not None else None
    if bucket is not None and graphs.batch is not None and bucket in graphs.graphs:
        return _consume_batched(graphs, slots, logits, tokens, count, bucket)
    for slot in slots:
        slot._settle()
    active = [(i, slots[i]) for i in range(count) if not slots[i].idle]
    queued = [(i, slot) for i, slot in active if slot.stageable()]
    handles = {}
    for i, slot in queued:
        graph = graphs.graphs.get((bucket, i)) if bucket is not None else None
        handles[i] = slot.stage(logits[i], tokens[i], graph)
    results = {i: slot.consume(logits[i], tokens[i]) for i, slot in active if i not in handles}
    results.update({i: slot.collect(handles[i]) for i, slot in queued})
    return {i: results[i] for i in sorted(results)}


def _consume_batched(graphs, slots, logits, tokens, count, bucket):
    """consume_batch over a PhiloxBatch: one host-to-device copy of every window's step scalars, one graph replay
    that selects and samples the bucket's windows, one device-to-host copy of their drawn classes and flags, and the
    host bookkeeping per slot from the copied rows (marking and finishing forwards still go through `consume`).
    The commits of steps that do not end their window are `DeferredCommit`s over the copied rows: the previous
    call's are settled first thing here (before this call's copy overwrites those rows), which in a loop that
    launches the next forward before calling this runs them while that forward is on the GPU."""
    batch = graphs.batch
    for commit in batch.pending:
        commit.materialize()
    batch.pending.clear()
    active = [(i, slots[i]) for i in range(count) if not slots[i].idle]
    queued = [(i, slot) for i, slot in active if slot.stageable()]
    B = batch.batch
    host = batch.host_scal.numpy()
    host[:] = 0
    frac = host[2 * B:3 * B].view(np.float64)
    for i, slot in queued:
        k, committed, f, step = slot.step_scalars()
        host[i], host[B + i], frac[i], host[3 * B + i] = k, committed, f, step
    batch.scal.copy_(batch.host_scal, non_blocking=True)
    graphs.graphs[bucket].replay()
    batch.host_drawn[:bucket].copy_(batch.drawn[:bucket].view(bucket, -1), non_blocking=True)
    batch.host_bad[:bucket].copy_(batch.sel.bad[:bucket].view(torch.uint8), non_blocking=True)
    batch.host_err.copy_(batch.err, non_blocking=True)
    event = torch.cuda.Event()
    event.record()
    staged = {i for i, _ in queued}
    results = {i: slot.consume(logits[i], tokens[i]) for i, slot in active if i not in staged}
    event.synchronize()
    if queued and int(batch.host_err[0]):
        raise RuntimeError('probability tensor contains either `inf`, `nan` or element < 0')
    drawn = batch.host_drawn.numpy()
    bad = batch.host_bad.numpy()
    for i, slot in queued:
        results[i] = slot.commit_drawn(drawn[i], bool(bad[i]), tokens[i], defer=True)
        if isinstance(results[i][1], DeferredCommit):
            batch.pending.append(results[i][1])
    return {i: results[i] for i in sorted(results)}
