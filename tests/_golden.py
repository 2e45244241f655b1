"""Loaders for the golden vectors in tests/golden/ (written by tests/golden/make_golden.py)."""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def _json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def quota_cases():
    """Yield dicts with score (fp32), selectable, non_last, order, chosen, k, b, frac, committed, name."""
    meta = _json('block_quota_select.json')
    data = np.load(os.path.join(GOLDEN, 'block_quota_select.npz'))
    for m in meta:
        shape = tuple(m['shape'])
        n = int(np.prod(shape))
        name = m['name']

        def bits(key):
            return np.unpackbits(data[name + '/' + key])[:n].astype(bool).reshape(shape)
        yield dict(name=name, shape=shape, b=m['b'], k=m['k'], frac=m['frac'], committed=m['committed'],
                   score=(data[name + '/score'].astype(np.float32) / np.float32(m['score_scale'])).reshape(shape),
                   selectable=bits('selectable'), non_last=bits('non_last'), chosen=bits('chosen'),
                   order=data[name + '/order'].astype(np.int64))


def schedule():
    return _json('schedule.json')


def lel_cases():
    meta = _json('lel_update.json')
    data = np.load(os.path.join(GOLDEN, 'lel_update.npz'))
    for m in meta:
        name = m['name']
        yield dict(m, **{k: data[name + '/' + k] for k in ('air', 'mask', 'solid', 'last0', 'out')})


def slot_cases():
    meta = _json('slot_trajectory.json')
    data = np.load(os.path.join(GOLDEN, 'slot_trajectory.npz'))
    for m in meta:
        name = m['name']
        yield dict(m, **{k: data[name + '/' + k] for k in ('step_map', 'values', 'tokens')})


def tiny_logits(step, shape, classes, ground):
    """The logits generator the slot trajectories were recorded with (torch CPU generator)."""
    import torch
    generator = torch.Generator().manual_seed(step + 1)
    logits = torch.randn((classes, *shape), generator=generator)
    logits[0, ground:] += 30.
    return logits


def hash_fill(shape, seed, scale=1.0):
    """Deterministic values in [-scale, scale) for the forward fixtures: splitmix64 of (index, seed), top 24 bits,
    u / 2^23 - 1, times `scale` (a power of two, so every value is exact in fp32 and fp64). The fixture script and
    the tests draw weights and inputs from it by name, so the vectors carry no weights."""
    n = int(np.prod(shape)) if len(shape) else 1
    with np.errstate(over='ignore'):
        z = np.arange(n, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(40)).astype(np.float64)
    return ((u / 2.0 ** 23 - 1.0) * scale).reshape(shape)


def name_seed(name, salt=0):
    """A stable per-name seed (CRC-32 of the name) for hash_fill."""
    import zlib
    return zlib.crc32(name.encode()) + 7919 * salt


def forward_meta():
    return _json('forward.json')


def forward_arrays():
    return np.load(os.path.join(GOLDEN, 'forward.npz'))
