"""Write the golden input/output vectors under tests/golden/ from the reference implementation.

Run in the build container only (the reference checkout is not present where the tests run):

    python tests/golden/make_golden.py /root/reference [sampling|rope|forward]

It imports the reference's pure-torch sampling functions and slot state machine, on the CPU, for the functions that
closed forms, brute force and invariants do not pin literally:
  * block_quota_select (streamvoxel/sampling/block_quota.py:20-38) - which voxels, not just how many;
  * counts / low_entropy_last_quotas (streamvoxel/sampling/schedule.py:32-38, low_entropy_last.py:20-33);
  * low_entropy_last_update (streamvoxel/sampling/low_entropy_last.py:8-17) at the fp32 threshold;
  * LowEntropyLastSlot trajectories (streamvoxel/stream/slot.py:50-176);
  * AxialRoPE (streamvoxel/models/unconditional_md4.py:10-24) on bf16 activations - the exact bf16 bits, which
    depend on the module's rounding order;
  * UnconditionalBlock with non-zero AdaLN shifts / scales / gates and the affine block, the time encoding, and one
    step forward of a tiny CompactStreamingControlNet through its own forward (models/compact_controlnet.py,
    models/unconditional_md4*.py) - what the step's oracle composes, with every weight and the zero projections
    non-zero.
Only data is written (inputs and expected outputs); no reference source is copied.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))      # tests/: the fixtures' own fill helper (_golden.hash_fill)


def tie_state(seed, shape, b):
    """Tie-heavy mid-window selection state (half-integer scores, ragged per-column deferred tops)."""
    g = torch.Generator().manual_seed(seed)
    last = torch.zeros(shape, dtype=torch.bool)
    tops = torch.randint(min(4, shape[0] - 1), shape[0], shape[1:], generator=g)
    for z in range(shape[1]):
        for x in range(shape[2]):
            last[tops[z, x]:, z, x] = True
    non_last = ~last
    committed_mask = non_last & (torch.rand(shape, generator=g) < torch.rand((), generator=g))
    selectable = non_last & ~committed_mask
    k = int(torch.randint(1, max(2, int(selectable.sum())), (), generator=g))
    committed = int(committed_mask.sum())
    frac = (committed + k) / int(non_last.sum())
    blocks = int(np.prod(shape)) // b ** 3
    order = torch.randperm(blocks, generator=g)
    score = (torch.randn(shape, generator=g) * 2).round() / 2
    return score, selectable, k, order, frac, committed, non_last


def fresh_state(seed, shape, b, k):
    """Fresh window (nothing committed, nothing deferred), bimodal real-valued scores."""
    g = torch.Generator().manual_seed(seed)
    selectable = torch.ones(shape, dtype=torch.bool)
    blocks = int(np.prod(shape)) // b ** 3
    order = torch.randperm(blocks, generator=g)
    # Multiples of 1/256 (exact in fp32, stored as int16 codes): 70% confident, 30% uncertain.
    score = torch.where(torch.rand(shape, generator=g) < .7, -torch.randint(0, 64, shape, generator=g).float(),
                        -1024 - torch.randint(0, 256, shape, generator=g).float()) / 256
    frac = k / int(np.prod(shape))
    return score, selectable, k, order, frac, 0, selectable.clone()


def quota_cases(block_view, block_quota_select):
    cases = []
    for seed in range(25):
        cases.append(('tie16x8x8_b4_s%d' % seed, 4) + tie_state(seed, (16, 8, 8), 4))
    for seed in range(6):
        cases.append(('tie8x8x8_b2_s%d' % seed, 2) + tie_state(100 + seed, (8, 8, 8), 2))
    cases.append(('tie256x16x16_b4', 4) + tie_state(7, (256, 16, 16), 4))
    cases.append(('tie256x16x16_b16', 16) + tie_state(8, (256, 16, 16), 16))
    cases.append(('tie64x16x16_b1', 1) + tie_state(9, (64, 16, 16), 1))
    cases.append(('fresh256x16x16_b4_k2621', 4) + fresh_state(10, (256, 16, 16), 4, 2621))
    cases.append(('fresh256x16x16_b16_k2621', 16) + fresh_state(11, (256, 16, 16), 16, 2621))
    arrays = {}
    meta = []
    for name, b, score, selectable, k, order, frac, committed, non_last in cases:
        n_total = block_view(non_last.contiguous(), b).sum(1)
        chosen = block_quota_select(score, selectable, k, b, order, frac, n_total)
        scale = 2 if bool(torch.equal(score * 2, (score * 2).round())) else 256
        assert torch.equal(score * scale, (score * scale).round())
        arrays[name + '/score'] = (score * scale).to(torch.int16).numpy()
        arrays[name + '/selectable'] = np.packbits(selectable.numpy().reshape(-1))
        arrays[name + '/non_last'] = np.packbits(non_last.numpy().reshape(-1))
        arrays[name + '/order'] = order.numpy().astype(np.int32)
        arrays[name + '/chosen'] = np.packbits(chosen.numpy().reshape(-1))
        meta.append(dict(name=name, shape=list(score.shape), b=b, k=k, frac=frac, committed=committed,
                         score_scale=scale, chosen_count=int(chosen.sum())))
    np.savez_compressed(os.path.join(HERE, 'block_quota_select.npz'), **arrays)
    with open(os.path.join(HERE, 'block_quota_select.json'), 'w') as f:
        json.dump(meta, f, indent=1)


def schedule_cases(counts, low_entropy_last_quotas, actual_time):
    rows = []
    for total in (512, 1024, 4096, 65536):
        for steps in (1, 2, 4, 8, 25, 26, 32, 128):
            for schedule in ('linear', 'quartercos', 'halfcos', 'reversequarter', 'arccos', 'front2', 'power2'):
                spec = dict(steps=steps, schedule=schedule, rounding='positive')
                rows.append(dict(total=total, spec=spec, counts=counts(total, spec)))
            for schedule in ('linear', 'halfcos', 'reversequarter'):
                spec = dict(steps=steps, schedule=schedule, rounding='legacy')
                rows.append(dict(total=total, spec=spec, counts=counts(total, spec)))
    quotas = []
    for total, steps in ((1024, 8), (65536, 8), (65536, 25), (65536, 26), (65536, 128)):
        for n_last in (0, 1, 37, total // 16, total // 3, total // 2, total - 1, total):
            quotas.append(dict(total=total, steps=steps, n_last=n_last,
                               quotas=low_entropy_last_quotas(total, steps, n_last, 'quartercos')))
    times = [dict(f=f, t=actual_time(f)) for f in (0., 1e-6, .1, .25, .5, .75, .9, 1 - 1e-6, 1., 1.5, -.5)]
    with open(os.path.join(HERE, 'schedule.json'), 'w') as f:
        json.dump(dict(counts=rows, quotas=quotas, actual_time=times), f)


def lel_cases(low_entropy_last_update):
    arrays = {}
    meta = []
    g = torch.Generator().manual_seed(4)
    shape = (32, 4, 4)
    for eps in (1e-3, 1e-4):
        edge = torch.tensor(1 - eps, dtype=torch.float32)
        near = torch.stack([torch.nextafter(edge, torch.tensor(0.)), edge, torch.nextafter(edge, torch.tensor(2.))])
        for mode, (band, col) in dict(col=(False, True), layer=(False, False), band=(True, False)).items():
            for trial in range(3):
                air = torch.where(torch.rand(shape, generator=g) < .85, torch.ones(shape), torch.rand(shape, generator=g))
                air[:, 0, 0] = near[torch.randint(3, (shape[0],), generator=g)]    # threshold edge values
                air[shape[0] // 2:, 1, 1] = 1.                                    # clean high tail
                mask = torch.rand(shape, generator=g) < .9
                solid = torch.rand(shape, generator=g) < .03
                last0 = torch.zeros(shape if col else shape[:1], dtype=torch.bool)
                if trial == 2:
                    last0[-2:] = True
                out = low_entropy_last_update(last0, mask, air, solid, eps, band, col)
                name = '%s_eps%g_t%d' % (mode, eps, trial)
                arrays[name + '/air'] = air.numpy()
                arrays[name + '/mask'] = mask.numpy()
                arrays[name + '/solid'] = solid.numpy()
                arrays[name + '/last0'] = last0.numpy()
                arrays[name + '/out'] = out.numpy()
                meta.append(dict(name=name, eps=eps, band=band, col=col))
    np.savez_compressed(os.path.join(HERE, 'lel_update.npz'), **arrays)
    with open(os.path.join(HERE, 'lel_update.json'), 'w') as f:
        json.dump(meta, f, indent=1)


def tiny_logits(step, shape, classes, ground):
    generator = torch.Generator().manual_seed(step + 1)
    logits = torch.randn((classes, *shape), generator=generator)
    logits[0, ground:] += 30.
    return logits


def slot_cases(LowEntropyLastSlot):
    """Trajectories of the reference slot on the CPU; logits are regenerated from (step, shape, classes, ground)."""
    arrays = {}
    meta = []
    runs = [dict(shape=(16, 8, 8), classes=6, cap=8, block=4, eps=1e-3, seeds=[3, 11, 12345]),
            dict(shape=(64, 16, 16), classes=12, cap=13, block=4, eps=1e-4, seeds=[7]),
            dict(shape=(32, 16, 16), classes=8, cap=10, block=16, eps=1e-3, seeds=[5]),
            dict(shape=(16, 8, 8), classes=6, cap=6, block=2, eps=1e-3, seeds=[21])]
    for r, run in enumerate(runs):
        shape, classes = run['shape'], run['classes']
        for i, seed in enumerate(run['seeds']):
            slot = LowEntropyLastSlot(shape, classes, air_ids=(0,), air_token=0, last_eps=run['eps'],
                                      block_size=run['block'], device='cpu')
            tokens = torch.full(shape, classes, dtype=torch.long)
            ground = shape[0] // 2 + i
            slot.arm(seed, run['cap'] + i, (i, 0))
            step, commits, record = 0, [], None
            while record is None:
                logits = tiny_logits(step + 31 * i, shape, classes, ground)
                record, commit = slot.consume(logits, tokens)
                if commit is not None:
                    commits.append(dict(step=commit['step'], n=len(commit['positions'])))
                step += 1
                assert step < 200
            name = 'run%d_seed%d' % (r, seed)
            arrays[name + '/step_map'] = record['step_map'].numpy()
            arrays[name + '/values'] = record['values'].numpy()
            arrays[name + '/tokens'] = tokens.numpy().astype(np.int16)
            meta.append(dict(name=name, shape=list(shape), classes=classes, cap=run['cap'] + i, block=run['block'],
                             eps=run['eps'], seed=seed, index=i, ground=ground, nfe=record['nfe'],
                             actual=record['actual'], last_count=record['last_count'], forwards=step,
                             commits=commits))
    np.savez_compressed(os.path.join(HERE, 'slot_trajectory.npz'), **arrays)
    with open(os.path.join(HERE, 'slot_trajectory.json'), 'w') as f:
        json.dump(meta, f, indent=1)


def rope_cases(AxialRoPE):
    """bf16 activations [B,H,N,D] at fp32 patch-centre positions (multiples of 1/8 up to ~300, as the condition
    builder produces), through the reference module on the CPU."""
    arrays, meta = {}, []
    for case, (B, H, N, D, seed) in enumerate([(2, 3, 40, 48, 5), (1, 2, 33, 24, 6), (1, 1, 64, 96, 7)]):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
        positions = torch.randint(-64, 2400, (B, N, 3), generator=g).float() / 8
        module = AxialRoPE(D)
        out = module(x, positions)
        name = 'case%d' % case
        arrays[name + '/x'] = x.view(torch.int16).numpy()
        arrays[name + '/positions'] = positions.numpy()
        arrays[name + '/frequencies'] = module.frequencies.numpy()
        arrays[name + '/out'] = out.view(torch.int16).numpy()
        meta.append(dict(name=name, shape=[B, H, N, D], seed=seed))
    np.savez_compressed(os.path.join(HERE, 'axial_rope.npz'), **arrays)
    with open(os.path.join(HERE, 'axial_rope.json'), 'w') as f:
        json.dump(meta, f, indent=1)


FWD_SCALE = 2.0 ** -3        # weights in [-1/8, 1/8): exact in fp32 and fp64
FWD_SHAPE = (16, 8, 8)        # window of the step fixtures (patch 4: 4 x 2 x 2 patch tokens)


def _fill(module, prefix):
    """Every parameter of `module` from hash_fill by its prefixed name (buffers keep the module's values)."""
    from _golden import hash_fill, name_seed
    names = []
    with torch.no_grad():
        for name, p in module.named_parameters():
            p.copy_(torch.from_numpy(hash_fill(tuple(p.shape), name_seed(prefix + name), FWD_SCALE)).to(p.dtype))
            names.append([name, list(p.shape)])
    return names


def _positions(shape, seed, span):
    """Multiples of 1/8 in [-span, span) (exact in fp32)."""
    from _golden import hash_fill
    return torch.from_numpy(np.round(hash_fill(shape, seed, span) * 8) / 8)


def forward_cases(ada_block, affine_block, ada_dit, plain_dit, compact):
    """The forward of the streaming ControlNet's pieces from the reference modules, weights and inputs drawn from
    hash_fill by name: UnconditionalBlock with AdaLN (non-zero shifts, scales and gates) and the affine one, in
    float64; the time encoding of the time-conditioned model (its sinusoidal features are fp32 in the module, so
    the model runs in fp32); and one step of a tiny CompactStreamingControlNet (5 x 48 backbone, 3 x 24 control,
    4 heads, a 16 x 8 x 8 window of 3 classes) through its own forward (the unpadded reference of the slot
    engines, stream/engine.py:87-102) in three variants: affine blocks (float64), time-free AdaLN (float64) and
    time-conditioned AdaLN (float32)."""
    from _golden import hash_fill, name_seed
    arrays, meta = {}, dict(blocks=[], step=[])
    W, H, N, B = 24, 2, 7, 2
    for kind, cls in (('ada', ada_block), ('affine', affine_block)):
        blk = cls(W, H, 4.0).double().eval()
        names = _fill(blk, f'block_{kind}.')
        x = torch.from_numpy(hash_fill((B, N, W), name_seed(f'block_{kind}.x'), 1.0))
        t = torch.from_numpy(hash_fill((B, W), name_seed(f'block_{kind}.t'), 1.0))
        pos = _positions((B, N, 3), name_seed(f'block_{kind}.pos'), 8.0)
        with torch.no_grad():
            out = blk(x, t, pos) if kind == 'ada' else blk(x, pos)
        arrays[f'block_{kind}/out'] = out.numpy()
        meta['blocks'].append(dict(kind=kind, width=W, heads=H, tokens=N, batch=B, params=names))
    # time encoding (fp32 module)
    dit = ada_dit(num_classes=3, voxel_shape=FWD_SHAPE, hidden_dim=48, depth=1, num_heads=4, time_dim=256).eval()
    names = _fill(dit, 'time.')
    ts = torch.tensor([0.0, 0.1, 0.37, 0.5, 0.999, 1.0])
    with torch.no_grad():
        arrays['time/out'] = dit.time_encoding(ts).double().numpy()
    meta['time'] = dict(t=ts.tolist(), time_dim=256, hidden=48,
                        params=[n for n in names if n[0].startswith(('time_mlp.', 'time_projection.'))])
    # one step of the tiny compact ControlNet
    C, P, L = 3, 5, 37
    for variant, dtype in (('affine', torch.float64), ('time_free', torch.float64), ('timed', torch.float32)):
        torch.manual_seed(0)
        if variant == 'affine':
            base = plain_dit(num_classes=C, voxel_shape=FWD_SHAPE, hidden_dim=48, depth=5, num_heads=4)
        else:
            base = ada_dit(num_classes=C, voxel_shape=FWD_SHAPE, hidden_dim=48, depth=5, num_heads=4,
                           time_free=variant == 'time_free')
        model = compact(base, control_depth=3, control_hidden_dim=24, checkpointing=False, biome_halo=4,
                        biome_patch=2, struct_classes=0).to(dtype).eval()
        names = _fill(model, f'step_{variant}.')
        pre = f'step_{variant}.'
        u = hash_fill((1, *FWD_SHAPE), name_seed(pre + 'tokens'), 1.0)
        tokens = torch.from_numpy(np.minimum(np.floor((u + 1.0) * 2.0), 3).astype(np.int64))
        heads, cw = 4, 24
        prefix = [(torch.from_numpy(hash_fill((1, heads, P, cw // heads), name_seed(pre + f'pk{j}'), 1.0)).to(dtype),
                   torch.from_numpy(hash_fill((1, heads, P, cw // heads), name_seed(pre + f'pv{j}'), 1.0)).to(dtype))
                  for j in range(3)]
        local = torch.from_numpy(hash_fill((1, L, cw), name_seed(pre + 'local'), 1.0)).to(dtype)
        lpos = _positions((1, L, 3), name_seed(pre + 'local_pos'), 16.0).to(dtype)
        t = torch.tensor([0.37])
        origin = torch.tensor([[16.0, -48.0, 8.0]], dtype=dtype)
        group = torch.tensor([0.0, -64.0, 0.0], dtype=dtype)
        with torch.no_grad():
            out = model(tokens, timestep=t, origin_xyz=origin, group_origin_xyz=group, prefix_kv=prefix, local=local,
                        local_positions=lpos)
        arrays[f'step_{variant}/out'] = out.double().numpy()
        arrays[f'step_{variant}/patch_centers_xyz'] = model.backbone.patch_centers_xyz.double().numpy()
        keep = [n for n in names if n[0].split('.')[0] in ('backbone', 'control', 'cross', 'zero')]
        meta['step'].append(dict(variant=variant, dtype=str(dtype).replace('torch.', ''), classes=C, prefix=P,
                                 local=L, depth=5, heads=heads, control_heads=heads, width=48, control_width=cw,
                                 layer_map={str(k): v for k, v in model.layer_map.items()}, patch=4,
                                 y_range=list(model.backbone.y_range), time_dim=256, voxel_shape=list(FWD_SHAPE),
                                 timestep=t.tolist(), origin=origin.tolist(), group_origin=group.tolist(),
                                 params=keep))
    np.savez_compressed(os.path.join(HERE, 'forward.npz'), **arrays)
    with open(os.path.join(HERE, 'forward.json'), 'w') as f:
        json.dump(meta, f)


def main(reference, only=None):
    sys.path.insert(0, reference)
    from streamvoxel.sampling.block_quota import block_quota_select, block_view
    from streamvoxel.sampling.low_entropy_last import low_entropy_last_quotas, low_entropy_last_update
    from streamvoxel.sampling.schedule import actual_time, counts
    from streamvoxel.stream.slot import LowEntropyLastSlot
    from streamvoxel.models.unconditional_md4 import AxialRoPE
    torch.set_num_threads(1)
    if only in (None, 'sampling'):
        quota_cases(block_view, block_quota_select)
        schedule_cases(counts, low_entropy_last_quotas, actual_time)
        lel_cases(low_entropy_last_update)
        slot_cases(LowEntropyLastSlot)
    if only in (None, 'rope'):
        rope_cases(AxialRoPE)
    if only in (None, 'forward'):
        from streamvoxel.models.compact_controlnet import CompactStreamingControlNet
        from streamvoxel.models.unconditional_md4 import UnconditionalBlock as AffineBlock
        from streamvoxel.models.unconditional_md4 import UnconditionalMD4DiT as PlainDiT
        from streamvoxel.models.unconditional_md4_timefree import UnconditionalBlock as AdaBlock
        from streamvoxel.models.unconditional_md4_timefree import UnconditionalMD4DiT as AdaDiT
        forward_cases(AdaBlock, AffineBlock, AdaDiT, PlainDiT, CompactStreamingControlNet)
    with open(os.path.join(HERE, 'provenance.json'), 'w') as f:
        json.dump(dict(torch=torch.__version__, numpy=np.__version__, reference=reference,
                       script='tests/golden/make_golden.py'), f, indent=1)


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference', sys.argv[2] if len(sys.argv) > 2 else None)
