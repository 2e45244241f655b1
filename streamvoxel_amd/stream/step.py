"""Static-buffer engines for one generation step of a batch of windows, capturable in a single HIP graph.

`CachedContext` holds the per-layer cross-attention K/V of every window (written once per window, read by every
step), `EaseSelect` the selection state of every window; `EaseSelect.run` is the whole EASE selection of a solid
step for all windows in one call (no host synchronisation), `EaseSelect.mark` the low-entropy-last marking pass.

Reference counterparts: PackedKeys / FastSlotForward._write (streamvoxel/stream/fast_ops.py:122-159, 241-250) for
the key store; FastLowEntropyLastSlot.prepare/select and SelectGraphs (streamvoxel/stream/fast_ops.py:519-540,
584-623) for the selection, which the reference captures as one graph per (bucket, slot); here one launch covers
all slots of the batch.
"""
from __future__ import annotations

import torch

from streamvoxel_amd import _lib
from streamvoxel_amd.stream.patches import PatchLogits
from streamvoxel_amd.sampling.block_quota import QuotaWorkspace, block_view
from streamvoxel_amd.stream.attention import attention

KEY_BLOCK = 64


class CachedContext:
    """Per-layer K [B,H,Kcap,D] and V (stored transposed, [B,H,D,Kcap]) with per-window lengths.

    Valid keys of window b are [0, L_b); the tail is zeroed on write. kv_dtype 'bf16' or 'fp8' (OCP e4m3fn with
    per-(window, head) scales); an fp8 cache is attended with the softmax weights in `p_dtype` ('bf16', the
    default: the reference's in-kernel dequantisation, within 5e-2 of fp32 attention over the unquantised K/V; or
    'e4m3': the fp8 matrix cores, an opt-in outside that bar; see `attention`)."""

    def __init__(self, layers, batch, heads, head_dim, kv_cap, device, kv_dtype='bf16', p_dtype='bf16'):
        if kv_dtype not in ('bf16', 'fp8'):
            raise ValueError("kv_dtype must be 'bf16' or 'fp8'")
        if p_dtype not in ('e4m3', 'bf16'):
            raise ValueError("p_dtype must be 'e4m3' or 'bf16'")
        self.p_dtype = p_dtype
        self.layers, self.batch, self.heads, self.head_dim = layers, batch, heads, head_dim
        self.kv_cap = kv_cap + (-kv_cap) % KEY_BLOCK
        self.kv_dtype = kv_dtype
        dt = torch.bfloat16 if kv_dtype == 'bf16' else torch.float8_e4m3fn
        self.k = [torch.zeros(batch, heads, self.kv_cap, head_dim, dtype=dt, device=device) for _ in range(layers)]
        self.vt = [torch.zeros(batch, heads, head_dim, self.kv_cap, dtype=dt, device=device) for _ in range(layers)]
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self.host_lengths = [0] * batch
        if kv_dtype == 'fp8':
            self.k_scale = [torch.ones(batch, heads, dtype=torch.float32, device=device) for _ in range(layers)]
            self.v_scale = [torch.ones(batch, heads, dtype=torch.float32, device=device) for _ in range(layers)]
        else:
            self.k_scale = self.v_scale = [None] * layers
        self._kv_ws = None

    def write(self, layer, index, key, value, prefix=None, positions=None, frequencies=None):
        """Window `index` of `layer` (FastSlotForward.encode + _write, fast_ops.py:228-250) in one `svhip_kv_write`:
        keys [0, P) from `prefix` = (prefix_k, prefix_v) [H, P, D] (already rotated, optional), keys [P, P + L)
        from key, value [H, L, D] (the local projections; K rotated by AxialRoPE at fp32 positions [L, 3] with the
        fp32 `frequencies` buffer when given), zeros after; an e4m3 cache also gets its per-(window, head) scales.
        Inputs are taken as bf16 (the reference's autocast dtype). The window's length is set on the host when the
        last layer is written or the length changes."""
        dev = self.k[layer].device
        rows = lambda t: t.to(device=dev, dtype=torch.bfloat16) if t.stride(-1) == 1 else (
            t.to(device=dev, dtype=torch.bfloat16).contiguous())
        key, value = rows(key), rows(value)
        _lib.require_gpu(key, value)
        H, L, D = key.shape
        if H != self.heads or D != self.head_dim or value.shape != key.shape:
            raise ValueError('key / value must be [heads, L, head_dim] like the cache')
        if prefix is not None:
            pk, pv = rows(prefix[0]), rows(prefix[1])
            if pk.shape[0] != H or pk.shape[2] != D or pv.shape != pk.shape:
                raise ValueError('prefix K / V must be [heads, P, head_dim]')
            P = pk.shape[1]
        else:
            pk = pv = None
            P = 0
        if P + L > self.kv_cap:
            raise ValueError('Condition exceeds the slot capacity')
        pos = freq = None
        if positions is not None:
            if frequencies is None:
                raise ValueError('rotating the local keys needs the AxialRoPE frequencies')
            pos = positions.to(device=dev, dtype=torch.float32).contiguous()
            freq = frequencies.to(device=dev, dtype=torch.float32).contiguous()
            if pos.shape != (L, 3):
                raise ValueError('positions must be [L, 3]')
        k, vt = self.k[layer][index], self.vt[layer][index]          # [H, Kcap, D], [H, D, Kcap]
        fp8 = self.kv_dtype == 'fp8'
        code = _lib.SVHIP_FP8_E4M3 if fp8 else _lib.SVHIP_BF16
        kc, vc = (k.view(torch.uint8), vt.view(torch.uint8)) if fp8 else (k, vt)
        lib = _lib.load()
        ws = None
        if fp8:
            nbytes = int(lib.svhip_kv_write_workspace_bytes(H, self.kv_cap))
            if self._kv_ws is None or self._kv_ws.numel() < nbytes:
                self._kv_ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            ws = self._kv_ws
        ks = self.k_scale[layer][index] if fp8 else None
        vs = self.v_scale[layer][index] if fp8 else None
        _lib.check(lib.svhip_kv_write(
            _lib.ptr(pk), _lib.ptr(pv), P, pk.stride(0) if P else 0, pk.stride(1) if P else 0,
            pv.stride(0) if P else 0, pv.stride(1) if P else 0, _lib.ptr(key), _lib.ptr(value), L, key.stride(0),
            key.stride(1), value.stride(0), value.stride(1), _lib.ptr(pos), 3, _lib.ptr(freq), H, D, _lib.ptr(kc),
            kc.stride(0), kc.stride(1), _lib.ptr(vc), vc.stride(0), vc.stride(2), vc.stride(1), self.kv_cap, code,
            _lib.ptr(ks), _lib.ptr(vs), _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_of(key)),
            'svhip_kv_write')
        if layer == self.layers - 1 or self.host_lengths[index] != P + L:
            self.set_length(index, P + L)

    def set_length(self, index, length):
        self.host_lengths[index] = int(length)
        self.lengths[index] = int(length)

    def attend(self, layer, query, out=None, n=None):
        """Attention of `query` [n,H,Q,D] (bf16) over the cached keys of the first n windows."""
        n = self.batch if n is None else n
        vt = self.vt[layer][:n].transpose(2, 3)
        ks = self.k_scale[layer]
        vs = self.v_scale[layer]
        return attention(query, self.k[layer][:n], vt, lengths=self.lengths[:n], out=out,
                         k_scale=None if ks is None else ks[:n], v_scale=None if vs is None else vs[:n],
                         p_dtype=self.p_dtype)


class EaseSelect:
    """Selection state of `batch` windows of `shape` ([Y,Z,X]) with `classes` classes and block size `block`.

    Buffers (all device, fixed addresses so that `run` / `mark` can be captured):
      tokens int64 [B,N] (mask token = classes), last bool [B,N], k / committed int64 [B], frac float64 [B],
      pos / n_total int64 [B,nb], chosen bool [B,N], bad bool [B], scores fp32 [B,N], air fp32 [B,N]."""

    def __init__(self, batch, shape, classes, block, device, air_ids=(0,)):
        self.batch, self.shape, self.classes, self.block = batch, tuple(shape), classes, block
        Y, Z, X = shape
        self.n = Y * Z * X
        self.nb = self.n // block ** 3
        dev = torch.device(device)
        self.device = dev
        self.tokens = torch.full((batch, self.n), classes, dtype=torch.int64, device=dev)
        self.last = torch.zeros((batch, self.n), dtype=torch.bool, device=dev)
        self.k = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.committed = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.frac = torch.zeros(batch, dtype=torch.float64, device=dev)
        self.pos = torch.zeros((batch, self.nb), dtype=torch.int64, device=dev)
        self.n_total = torch.zeros((batch, self.nb), dtype=torch.int64, device=dev)
        self.chosen = torch.zeros((batch, self.n), dtype=torch.bool, device=dev)
        self.bad = torch.zeros(batch, dtype=torch.bool, device=dev)
        self.scores = torch.zeros((batch, self.n), dtype=torch.float32, device=dev)
        self.air = torch.zeros((batch, self.n), dtype=torch.float32, device=dev)
        self.air_index = torch.as_tensor(list(air_ids), dtype=torch.int32, device=dev)
        self.ws = QuotaWorkspace(batch, self.shape, block, dev, fused=True)

    @staticmethod
    def _layout(logits, batch, n):
        """(dtype code, classes, stride_b, stride_c, stride_n) for [B,C,Y,Z,X] / [B,C,N] class-major or
        [B*N, C] / [B,N,C] voxel-major logits."""
        if logits.dim() == 2:                        # [B*N, C] voxel-major
            C = logits.shape[1]
            return _lib.dtype_code(logits.dtype), C, n * logits.stride(0), logits.stride(1), logits.stride(0)
        if logits.dim() == 3 and logits.shape[1] == n:   # [B, N, C]
            return (_lib.dtype_code(logits.dtype), logits.shape[2], logits.stride(0), logits.stride(2),
                    logits.stride(1))
        x = logits.reshape(logits.shape[0], logits.shape[1], -1)   # [B, C, N] class-major
        if x.data_ptr() != logits.data_ptr():
            raise ValueError('class-major logits must flatten to [B, C, N] without a copy')
        return _lib.dtype_code(x.dtype), x.shape[1], x.stride(0), x.stride(1), x.stride(2)

    def bind_window(self, index, order, last=None):
        """Once per window (FastLowEntropyLastSlot.prepare's `_bound` part, fast_ops.py:524-528): the deferred
        mask, per-block non-deferred counts and the inverse block order of window `index`."""
        if last is not None:
            self.last[index].copy_(last.reshape(-1))
        lv = self.last[index].reshape(self.shape)
        self.n_total[index].copy_(block_view((~lv).contiguous(), self.block).sum(1))
        self.pos[index][order.to(self.device)] = torch.arange(self.nb, device=self.device)

    def set_step(self, index, k, committed, frac):
        """Per-step scalars of window `index` (host numbers; device fills, no host read)."""
        self.k[index].fill_(int(k))
        self.committed[index].fill_(int(committed))
        self.frac[index].fill_(float(frac))

    def _patch_rows(self, logits):
        if logits.shape != self.shape:
            raise ValueError(f'patch logits of {logits.shape} windows, the selection is for {self.shape}')
        return logits.rows

    def run(self, logits, n=None, keep_scores=False, scalars=None):
        """Entropy + selectable + block-quota select + bad flag for the first n windows (capturable). With
        keep_scores the fp32 scores are also left in `self.scores`. `logits` may be a PatchLogits (the class
        head's output read in place). `scalars`: the windows' (k, committed, frac) as device tensors of at least
        n entries (int64, int64, float64) to read in place of this selection's own buffers (`set_step`), e.g. a
        row of per-step tables that a captured step reads directly."""
        n = self.batch if n is None else n
        Y, Z, X = self.shape
        lib = _lib.load()
        k, committed, frac = self.k, self.committed, self.frac
        if scalars is not None:
            k, committed, frac = scalars
            for t, dtype, name in ((k, torch.int64, 'k'), (committed, torch.int64, 'committed'),
                                   (frac, torch.float64, 'frac')):
                if not (torch.is_tensor(t) and t.device == self.k.device and t.dtype == dtype and t.dim() == 1
                        and t.numel() >= n and t.is_contiguous()):
                    raise ValueError(f'scalars: {name} must be a contiguous {dtype} device vector of at least {n}')
        if isinstance(logits, PatchLogits):
            rows = self._patch_rows(logits)
            _lib.require_gpu(rows)
            _lib.check(lib.svhip_ease_select_patches(
                _lib.ptr(rows), _lib.dtype_code(rows.dtype), logits.classes, logits.patch, rows.stride(0),
                rows.stride(1), _lib.ptr(self.tokens), self.classes, _lib.ptr(self.last.view(torch.uint8)), n, Y, Z,
                X, self.block, _lib.ptr(k), _lib.ptr(self.pos), _lib.ptr(frac), _lib.ptr(self.n_total),
                _lib.ptr(committed), _lib.ptr(self.chosen.view(torch.uint8)), _lib.ptr(self.bad.view(torch.uint8)),
                _lib.ptr(self.scores) if keep_scores else None, _lib.ptr(self.ws.buffer), self.ws.buffer.numel(),
                _lib.stream_of(rows)), 'svhip_ease_select_patches')
            return
        _lib.require_gpu(logits)
        code, C, sb, sc, sn = self._layout(logits, n, self.n)
        _lib.check(lib.svhip_ease_select(
            _lib.ptr(logits), code, C, sb, sc, sn, _lib.ptr(self.tokens), self.classes,
            _lib.ptr(self.last.view(torch.uint8)), n, Y, Z, X, self.block, _lib.ptr(k), _lib.ptr(self.pos),
            _lib.ptr(frac), _lib.ptr(self.n_total), _lib.ptr(committed),
            _lib.ptr(self.chosen.view(torch.uint8)), _lib.ptr(self.bad.view(torch.uint8)),
            _lib.ptr(self.scores) if keep_scores else None,
            _lib.ptr(self.ws.buffer), self.ws.buffer.numel(), _lib.stream_of(logits)), 'svhip_ease_select')

    def mark(self, logits, eps, n=None):
        """Low-entropy-last marking pass (stream/slot.py:124-129): air probability of every voxel and the
        per-column top run of certain air OR-ed into `last` (capturable; the deferred count is read later)."""
        n = self.batch if n is None else n
        Y, Z, X = self.shape
        lib = _lib.load()
        if isinstance(logits, PatchLogits):
            rows = self._patch_rows(logits)
            _lib.require_gpu(rows)
            stream = _lib.stream_of(rows)
            _lib.check(lib.svhip_air_prob_patches(
                _lib.ptr(rows), _lib.dtype_code(rows.dtype), n, logits.classes, Y, Z, X, logits.patch, rows.stride(0),
                rows.stride(1), _lib.ptr(self.air_index), int(self.air_index.numel()), _lib.ptr(self.air), stream),
                'svhip_air_prob_patches')
        else:
            code, C, sb, sc, sn = self._layout(logits, n, self.n)
            stream = _lib.stream_of(logits)
            _lib.check(lib.svhip_air_prob(_lib.ptr(logits), code, n, C, self.n, sb, sc, sn, _lib.ptr(self.air_index),
                                          int(self.air_index.numel()), _lib.ptr(self.air), stream), 'svhip_air_prob')
        _lib.check(lib.svhip_lel_update(_lib.ptr(self.last.view(torch.uint8)), None, _lib.ptr(self.air), None,
                                        float(eps), _lib.SVHIP_LEL_COLUMN, n, Y, Z, X, stream), 'svhip_lel_update')
