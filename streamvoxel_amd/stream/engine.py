"""The slot engine: a batch of window slots, each with its cached cross-attention context, and one captured HIP
graph of the generation step per batch bucket.

Drop-in surface: the attributes and methods the reference's worker drives on `FastSlotForward`
(streamvoxel/stream/fast_ops.py:164-375, used at streamvoxel/stream/worker.py:269-280, 378-397): `tokens`, `shape`,
`batch`, `sizes`, `graphs`, `graph`, `outputs`, `packed`, `load_slot`, `wait_loads`, `clear_tokens`, `bucket`,
`replay(timesteps, count)`, `eager`, `numerical_gate`. What runs:

  * `load_slot(index, item)`: the window's condition, in the layout `encode_item` returns (prefix K/V per layer,
    already rotated; local context features and their positions), becomes the slot's cache entry on a side stream:
    the local K/V projection (the layer's torch Linear), then one `svhip_kv_write` per layer (prefix rows, local keys
    rotated by AxialRoPE, zeros to the capacity, bf16 or e4m3 with per-head scales). The encoders that turn an
    item into that condition are the model's and stay outside this library: pass them as `encoder`.
  * the step: `StepForward` (gather patchify, backbone and control blocks, cross attention over the cache, zero
    projections, final norm, class head) over the first n slots, returning the class head's rows in patch order
    (`PatchLogits`), which the slots' selection reads in place.
  * `StepGraphs` captures one graph per bucket size (1, 2, 4, ... and the batch), so a half-empty batch replays the
    smallest graph covering its leading slots. Capture failure leaves the engine eager and says so on stdout.
"""
from __future__ import annotations

import json
from typing import NamedTuple

import torch

from streamvoxel_amd.stream.forward import StepForward
from streamvoxel_amd.stream.step import CachedContext

__all__ = ['Encoded', 'StepGraphs', 'SlotEngine', 'condition_widths', 'write_condition', 'RECOMMENDED']

# The reference's recommended options (fast_ops.py:35); every combination runs the same kernels here.
RECOMMENDED = dict(patchify='gather', attention='flex', compile='emulate')


class Encoded(NamedTuple):
    """One window's condition as the reference's `encode_item` returns it (streamvoxel/stream/engine.py:77-87):
    `prefix` one (K, V) pair [H, P, D] per cross-attention layer (K already rotated, `encode_kv`), `local` the
    local context features [1, L, W] and `positions` their fp32 XYZ positions [1, L, 3]."""
    prefix: list
    local: torch.Tensor
    positions: torch.Tensor


def default_encoder(model, spec, device):
    """The encoder a worker gets when it passes none, as `worker.py:272` constructs `FastSlotForward`: for the
    reference's models (those with `encode_group`) the reference package's own `encode_item`
    (streamvoxel/stream/engine.py:75-87) when that package is importable, its (prefix, local, positions) as an
    `Encoded`; otherwise None (`load_slot` then takes an `Encoded` itself)."""
    if not hasattr(model, 'encode_group'):
        return None
    try:
        from streamvoxel.stream.engine import encode_item
    except ImportError:
        return None
    return lambda item: Encoded(*encode_item(model, item, spec, device))


def condition_widths(model, spec):
    """Tokens one L1 tile, one L2 tile and the biome window contribute (streamvoxel/stream/engine.py:62-74): an L1
    tile is its 4^3 patches, an L2 tile its 16^3 patches, the biome window (height/4) x 12 x 12 cells at halo 16
    and patch 1, otherwise a 6 (halo 4) or 12 cell square padded to the biome patch and pooled by it."""
    height, tile = int(spec.height), int(spec.tile)
    l1 = (height // 4) * (tile // 4) ** 2
    l2 = (height // 16) * (tile // 16) ** 2
    halo, patch = int(getattr(model, 'biome_halo', 16)), int(getattr(model, 'biome_patch', 1))
    if halo == 16 and patch == 1:
        biome = (height // 4) * 12 * 12
    else:
        side = 6 if halo == 4 else 12
        side += (-side) % patch
        biome = (height // 4 // patch) * (side // patch) ** 2
    return l1, l2, biome


def buckets(batch):
    """Captured batch sizes: the powers of two below `batch`, then `batch` itself."""
    sizes, n = [], 1
    while n < batch:
        sizes.append(n)
        n *= 2
    return sizes + [batch]


def write_condition(model, context, index, enc):
    """Every layer's cache entry of slot `index` of `context` (FastSlotForward.encode + _write, fast_ops.py:228-250):
    local K / V = the layer's key_value projection of `enc.local` (bf16 autocast, as the reference's), local K
    rotated at `enc.positions` by `svhip_kv_write`, the prefix rows first, zeros to the capacity."""
    dev = context.lengths.device
    local = enc.local.to(dev)
    positions = enc.positions.to(device=dev, dtype=torch.float32)[0]
    L = local.shape[1]
    with torch.autocast('cuda', dtype=torch.bfloat16):
        for j, cross in enumerate(model.cross):
            H = int(cross.heads)
            D = int(cross.width) // H
            kv = cross.key_value(local[0]).to(torch.bfloat16).view(L, 2, H, D)
            key, value = kv[:, 0].transpose(0, 1), kv[:, 1].transpose(0, 1)      # [H, L, D] views
            pk, pv = enc.prefix[j]
            context.write(j, index, key, value, prefix=(pk, pv), positions=positions,
                          frequencies=cross.rope.frequencies)


class StepGraphs:
    """One captured HIP graph per key of a step body `body(key) -> output` on `device`.

    Every key's body runs `warmup` times on a side stream first (library handles and workspaces get made outside
    capture), then the keys are captured in the given order into one memory pool, each output kept alive in
    `outputs[key]`. Graphs sharing the pool must not run concurrently; replays of any order are fine because every
    output stays allocated. If a capture fails, `graphs` and `outputs` are emptied, `ok` is False, one JSON line
    reports the error, and `__call__` runs the body eagerly."""

    def __init__(self, device, body, keys, capture=True, warmup=2):
        self.device = torch.device(device)
        self.body = body
        self.keys = list(keys)
        self.graphs, self.outputs = {}, {}
        self.ok = False
        if capture:
            self._capture(warmup)

    def _capture(self, warmup):
        dev = self.device
        main = torch.cuda.current_stream(dev)
        warm = torch.cuda.Stream(device=dev)
        warm.wait_stream(main)
        with torch.cuda.stream(warm):
            for key in self.keys:
                for _ in range(warmup):
                    self.body(key)
        main.wait_stream(warm)
        torch.cuda.synchronize(dev)
        # A capture stream of this device's own: torch's default capture stream belongs to the first device that
        # captured.
        stream = torch.cuda.Stream(device=dev)
        pool = torch.cuda.graph_pool_handle()
        try:
            for key in self.keys:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=pool, stream=stream, capture_error_mode='thread_local'):
                    out = self.body(key)
                self.graphs[key] = graph
                self.outputs[key] = out
            self.ok = True
        except Exception as error:   # the engine stays usable eagerly, as the reference's does
            self.graphs, self.outputs = {}, {}
            self.ok = False
            print(json.dumps(dict(event='hip_graph_fallback', device=str(dev),
                                  error=f'{type(error).__name__}: {error}')), flush=True)

    def __call__(self, key):
        graph = self.graphs.get(key)
        if graph is None:
            return self.body(key)
        graph.replay()
        return self.outputs[key]


PATCHIFY = ('gather', 'conv')
ATTENTION = ('flex', 'sdpa')
KV_DTYPES = ('bf16', 'fp8')


def check_engine_options(patchify, attention, compile, kv_dtype='bf16'):
    """The engine's options, validated as the reference does (fast_ops.py:170-171): ValueError for unknown ones."""
    if patchify not in PATCHIFY or attention not in ATTENTION:
        raise ValueError('patchify must be gather|conv and attention flex|sdpa')
    if compile not in (False, True, 'emulate'):
        raise ValueError("compile must be False, True or 'emulate'")
    if kv_dtype not in KV_DTYPES:
        raise ValueError(f'kv_dtype must be one of {KV_DTYPES}')


class SlotEngine:
    """`batch` window slots of the model `model` (the reference's StreamingControlNet / CompactStreamingControlNet,
    or a module with the same attributes: backbone, control, cross, zero, optional layer_map) for windows of
    spec.height x spec.tile x spec.tile voxels and spec.num_classes classes, on a HIP device.

    Capacity per slot: l2_cap L2 tiles of prefix keys and l1_cap L1 tiles plus the biome window of local keys
    (`condition_widths`), rounded up to the kernel's 64-key block. `encoder(item) -> Encoded` turns a scheduler
    item into the condition (for the reference's model: `lambda item: encode_item(model, item, spec, device)`, which
    `default_encoder` supplies when none is passed and the reference's package is importable); without one,
    `load_slot` takes an `Encoded` (or a (prefix, local, positions) tuple) itself.
    `kv_dtype` 'bf16' (the reference's cache) or 'fp8' (e4m3 with per-(window, head) scales). `concurrent` runs the
    control branch on its own stream inside the step. `patchify`, `attention` and `compile` are the reference's
    option names (fast_ops.py:168-171): 'gather' and 'conv' both run the HIP gather patchify, bit for bit the
    reference's embedding-bag form, which computes the one-hot Conv3d's sum (the reference's own test,
    tests/stream/test_live_fast_ops.py:14-21, holds the two equal); 'flex' and 'sdpa' both run the HIP attention
    kernel over the slots' key lengths (each is masked attention over the valid keys); `compile` is accepted and
    changes nothing (the blocks run on HIP kernels that round where eager autocast does)."""

    def __init__(self, model, spec, device, batch, l1_cap, l2_cap, *, patchify='gather', attention='flex',
                 compile=False, capture=True, encoder=None, kv_dtype='bf16', concurrent=True):
        check_engine_options(patchify, attention, compile, kv_dtype)
        self.device = torch.device(device)
        if self.device.type != 'cuda':
            raise RuntimeError('SlotEngine runs on a HIP device; there is no CPU path')
        if self.device.index is None:
            self.device = torch.device('cuda', torch.cuda.current_device())
        self.model, self.spec = model, spec
        self.encoder = encoder if encoder is not None else default_encoder(model, spec, self.device)
        self.batch, self.l1_cap, self.l2_cap = int(batch), int(l1_cap), int(l2_cap)
        if self.batch < 1:
            raise ValueError('batch must be at least 1')
        self.classes = int(spec.num_classes)
        self.shape = (int(spec.height), int(spec.tile), int(spec.tile))
        self.options = dict(patchify=patchify, attention=attention, compile=compile, kv_dtype=kv_dtype)
        self.l1_tokens, self.l2_tokens, self.biome_tokens = condition_widths(model, spec)
        self.prefix_len = self.l2_cap * self.l2_tokens
        self.local_len = self.l1_cap * self.l1_tokens + self.biome_tokens
        cross = model.cross[0]
        heads = int(cross.heads)
        dev = self.device
        self.context = CachedContext(len(model.cross), self.batch, heads, int(cross.width) // heads,
                                     self.prefix_len + self.local_len, dev, kv_dtype)
        self.forward_fn = StepForward(model, self.context, concurrent=concurrent)
        self.tokens = torch.full((self.batch, *self.shape), self.classes, dtype=torch.int64, device=dev)
        self.timestep = torch.ones(self.batch, dtype=torch.float32, device=dev)
        self.group_origin = torch.tensor([0.0, float(getattr(spec, 'y_origin', 0.0)), 0.0], device=dev)
        self.origin = self.group_origin.expand(self.batch, 3).contiguous()
        self.side = torch.cuda.Stream(device=dev)
        self.sizes = buckets(self.batch)
        # Largest first, so the full batch's intermediates are the pool's first tenants.
        self.steps = StepGraphs(dev, self.forward, sorted(self.sizes, reverse=True), capture=capture)
        self.graph = self.graphs.get(self.batch)

    # -- the reference's attribute names
    @property
    def graphs(self):
        return self.steps.graphs

    @property
    def outputs(self):
        return self.steps.outputs

    @property
    def graph_ok(self):
        return self.steps.ok

    @property
    def packed(self):
        """The cache (`PackedKeys` in the reference): per-layer K / V^T, `lengths` int32 [batch]."""
        return self.context

    # -- conditions
    def encode(self, item):
        """The slot condition of `item`: the encoder's output, or `item` itself when there is no encoder."""
        enc = self.encoder(item) if self.encoder is not None else item
        if not isinstance(enc, Encoded):
            prefix, local, positions = enc
            enc = Encoded(list(prefix), local, positions)
        if len(enc.prefix) != self.context.layers:
            raise ValueError(f'the condition has {len(enc.prefix)} prefix layers, the model {self.context.layers}')
        if enc.local.dim() != 3 or enc.local.shape[0] != 1 or enc.positions.shape != (1, enc.local.shape[1], 3):
            raise ValueError('local must be [1, L, W] with positions [1, L, 3]')
        P = enc.prefix[0][0].shape[1] if len(enc.prefix) else 0
        if P > self.prefix_len or enc.local.shape[1] > self.local_len:
            raise ValueError('Condition exceeds the slot capacity')
        return enc

    @torch.inference_mode()
    def load_slot(self, index, item):
        """Slot `index` takes `item`'s condition and a fresh (all-mask) token state, enqueued on the side stream;
        `wait_loads` joins it before the next replay. The side stream first waits for the current stream, so a
        step still reading the slot's cache finishes before the cache is overwritten."""
        index = int(index)
        if not 0 <= index < self.batch:
            raise IndexError(f'slot {index} of {self.batch}')
        main = torch.cuda.current_stream(self.device)
        self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            enc = self.encode(item)
            for t in (enc.local, enc.positions, *[x for pair in enc.prefix for x in pair]):
                if torch.is_tensor(t) and t.is_cuda:
                    t.record_stream(self.side)
            write_condition(self.model, self.context, index, enc)
            self.tokens[index].fill_(self.classes)

    def wait_loads(self):
        torch.cuda.current_stream(self.device).wait_stream(self.side)

    def clear_tokens(self):
        self.wait_loads()
        self.tokens.fill_(self.classes)

    def bucket(self, count):
        """The smallest captured size covering the first `count` slots."""
        count = max(1, int(count))
        for size in self.sizes:
            if size >= count:
                return size
        raise ValueError(f'{count} slots of a batch of {self.batch}')

    # -- the step
    def forward(self, n):
        """The step's forward over the first n slots -> PatchLogits [n] (class head rows in patch order)."""
        return self.forward_fn(self.tokens[:n], self.timestep[:n], self.origin[:n], self.group_origin)

    def _set_time(self, timestep):
        t = torch.as_tensor(timestep, dtype=torch.float32).reshape(-1)
        if t.numel() == 1:
            self.timestep.fill_(float(t))
        else:
            if t.numel() != self.batch:
                raise ValueError(f'{t.numel()} timesteps for {self.batch} slots')
            self.timestep.copy_(t)

    def replay(self, timestep, count=None):
        """Logits of the first `bucket(count)` slots (all slots when count is None) at `timestep` (one per slot,
        or one for all): a graph replay, or the eager step if no graph was captured."""
        self._set_time(timestep)
        return self.steps(self.batch if count is None else self.bucket(count))

    def eager(self, timestep):
        self._set_time(timestep)
        return self.forward(self.batch)

    # -- the numerical gate
    def _reference_logits(self, item):
        """Class-major logits [1, C, Y, Z, X] of `item` at timestep 1 from an independent path: the model's own
        forward over the unpadded condition when the model has one (the reference's `unpadded_logits`,
        streamvoxel/stream/engine.py:87-102), else this library's step on a one-slot cache sized to the
        condition alone (no padding beyond the 64-key block) and captured nowhere."""
        enc = self.encode(item)
        dev = self.device
        tokens = torch.full((1, *self.shape), self.classes, dtype=torch.int64, device=dev)
        time = torch.ones(1, device=dev)
        if type(self.model).forward is not torch.nn.Module.forward:
            stacked = [(k.to(dev)[None], v.to(dev)[None]) for k, v in enc.prefix]
            with torch.inference_mode(), torch.autocast('cuda', dtype=torch.bfloat16):
                out = self.model(tokens, timestep=time, origin_xyz=self.origin[:1], group_origin_xyz=self.group_origin,
                                 prefix_kv=stacked, local=enc.local.to(dev), local_positions=enc.positions.to(dev))
            return out, 'model_forward'
        length = (enc.prefix[0][0].shape[1] if len(enc.prefix) else 0) + enc.local.shape[1]
        ctx = CachedContext(self.context.layers, 1, self.context.heads, self.context.head_dim, max(length, 1), dev,
                            self.context.kv_dtype)
        write_condition(self.model, ctx, 0, enc)
        step = StepForward(self.model, ctx, concurrent=False)
        out = step(tokens, time, self.origin[:1], self.group_origin)
        return out.class_major(), 'one_slot_exact_cache'

    @torch.inference_mode()
    def numerical_gate(self, item, other=None):
        """The reference's gate report (fast_ops.py:351-375): slot 0 (and 1) take `item` (and `other`); the eager
        step against its graph replay (bit-identical), against the independent reference logits (argmax agreement
        >= 0.999 and mean |difference| <= 0.05) and the two-slot bucket against the full batch (the same bar).
        Slots 0 and 1 keep these conditions afterwards."""
        reference, source = self._reference_logits(item)
        reference = reference.float()
        self.load_slot(0, item)
        if other is not None and self.batch > 1:
            self.load_slot(1, other)
        self.wait_loads()
        time = torch.ones(self.batch)
        eager = self.eager(time).class_major().clone()
        replayed = self.replay(time).class_major().clone() if self.graph is not None else eager
        equal = self.graph is not None and bool(torch.equal(eager, replayed))
        gap = (eager[0].float() - reference[0]).abs()
        match = float((eager[0].argmax(0) == reference[0].argmax(0)).float().mean())
        mean_abs = float(gap.mean())
        lead = min(2, self.batch)
        small = self.replay(time, lead).class_major()[:lead].float()
        bucket_match = float((small.argmax(1) == eager[:lead].argmax(1)).float().mean())
        bucket_close = bucket_match >= 0.999 and float((small - eager[:lead].float()).abs().mean()) <= 0.05
        return dict(graph_equal=equal, graph_used=self.graph is not None,
                    padded_close=bool(match >= 0.999 and mean_abs <= 0.05), bucket_close=bool(bucket_close),
                    bucket_match=bucket_match, buckets=sorted(self.graphs) or [], max_abs=float(gap.max()),
                    mean_abs=mean_abs, argmax_match=match, batch=self.batch, prefix_len=self.prefix_len,
                    local_len=self.local_len, options=self.options, reference=source)
