"""Pins of the transformer-block oracle (oracle/backbone.py) by closed forms and invariants, on the CPU."""
import math

import numpy as np

import torch

from oracle import attention as A
from oracle import backbone as O
from oracle import producer as P

F64 = torch.float64


def test_layer_norm_invariants_and_affine():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 40, generator=g, dtype=F64) * 3 + 7
    eps = 1e-6
    y = O.layer_norm(x, eps)
    var = x.var(-1, unbiased=False, keepdim=True)
    assert torch.allclose(y.mean(-1), torch.zeros(3, 5, dtype=F64), atol=1e-12)
    # biased variance: var(y) = var / (var + eps) exactly (an unbiased divisor would fail this)
    assert torch.allclose(y.var(-1, unbiased=False, keepdim=True), var / (var + eps), rtol=1e-12)
    w, b = torch.randn(40, generator=g, dtype=F64), torch.randn(40, generator=g, dtype=F64)
    assert torch.allclose(O.layer_norm(x, eps, w, b), y * w + b, rtol=1e-13, atol=1e-13)
    # a large eps pulls the output towards zero by sqrt(var / (var + eps))
    y2 = O.layer_norm(x, 100.0)
    assert torch.allclose(y2, y * torch.sqrt((var + eps) / (var + 100.0)), rtol=1e-12)


def test_modulate_closed_form():
    x = torch.tensor([[[1.0, -2.0], [0.5, 4.0]]], dtype=F64)          # [1, 2, 2]
    shift = torch.tensor([[10.0, 20.0]], dtype=F64)
    scale = torch.tensor([[1.0, -0.5]], dtype=F64)
    want = torch.tensor([[[12.0, 19.0], [11.0, 22.0]]], dtype=F64)
    assert torch.equal(O.modulate(x, shift, scale), want)


def test_gelu_and_silu_known_values():
    x = torch.tensor([-1.0, 0.0, 1.0], dtype=F64)
    assert torch.allclose(O.gelu(x), torch.tensor([-0.15865525393145707, 0.0, 0.8413447460685429], dtype=F64),
                          rtol=0, atol=1e-15)
    assert torch.allclose(O.silu(x), torch.tensor([-0.2689414213699951, 0.0, 0.7310585786300049], dtype=F64),
                          rtol=0, atol=1e-15)
    t = torch.linspace(-6, 6, 97, dtype=F64)
    # odd parts: f(x) - f(-x) = x for both (x * Phi(x) and x * sigmoid(x))
    assert torch.allclose(O.gelu(t) - O.gelu(-t), t, atol=1e-14)
    assert torch.allclose(O.silu(t) - O.silu(-t), t, atol=1e-14)


def _attn_params(width, seed):
    g = torch.Generator().manual_seed(seed)
    return {
        'attn.qkv.weight': torch.randn(3 * width, width, generator=g, dtype=F64) / math.sqrt(width),
        'attn.qkv.bias': torch.randn(3 * width, generator=g, dtype=F64) * 0.1,
        'attn.proj.weight': torch.randn(width, width, generator=g, dtype=F64) / math.sqrt(width),
        'attn.proj.bias': torch.randn(width, generator=g, dtype=F64) * 0.1,
    }


def test_rotary_attention_uniform_scores_give_the_mean_of_v():
    """Q and K projections zero: every score is 0, so every token's output is proj(mean over tokens of V)."""
    B, N, W, H = 2, 7, 24, 2
    p = _attn_params(W, 1)
    p['attn.qkv.weight'][:2 * W] = 0
    p['attn.qkv.bias'][:2 * W] = 0
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, N, W, generator=g, dtype=F64)
    pos = torch.rand(B, N, 3, generator=g) * 10
    v = x @ p['attn.qkv.weight'][2 * W:].t() + p['attn.qkv.bias'][2 * W:]
    want = v.mean(1, keepdim=True) @ p['attn.proj.weight'].t() + p['attn.proj.bias']
    got = O.rotary_attention(x, pos, p, H)
    assert torch.allclose(got, want.expand(B, N, W), rtol=1e-12, atol=1e-12)


def test_rotary_attention_single_token_and_zero_positions():
    B, W, H = 3, 24, 2
    p = _attn_params(W, 3)
    g = torch.Generator().manual_seed(4)
    # one token: softmax over one key is 1, the output is proj(v) whatever the rotation
    x = torch.randn(B, 1, W, generator=g, dtype=F64)
    pos = torch.rand(B, 1, 3, generator=g) * 50
    v = x @ p['attn.qkv.weight'][2 * W:].t() + p['attn.qkv.bias'][2 * W:]
    want = v @ p['attn.proj.weight'].t() + p['attn.proj.bias']
    assert torch.allclose(O.rotary_attention(x, pos, p, H), want, rtol=1e-12, atol=1e-12)
    # positions 0: the rotation is the identity, so the result is plain attention on the [3, H, D] split
    N = 6
    x = torch.randn(B, N, W, generator=g, dtype=F64)
    qkv = (x @ p['attn.qkv.weight'].t() + p['attn.qkv.bias']).reshape(B, N, 3, H, W // H)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    o = A.cross_attention_bruteforce(q, k, v, [N] * B)
    want = o.transpose(1, 2).reshape(B, N, W) @ p['attn.proj.weight'].t() + p['attn.proj.bias']
    got = O.rotary_attention(x, torch.zeros(B, N, 3), p, H)
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)
    # and a rotation of both Q and K by the same phase everywhere leaves the scores unchanged
    same = torch.full((B, N, 3), 3.25)
    assert torch.allclose(O.rotary_attention(x, same, p, H), want, rtol=1e-6, atol=1e-6)


def _block_params(W, seed, timed):
    g = torch.Generator().manual_seed(seed)
    p = _attn_params(W, seed)
    p.update({
        'mlp.0.weight': torch.randn(4 * W, W, generator=g, dtype=F64) / math.sqrt(W),
        'mlp.0.bias': torch.randn(4 * W, generator=g, dtype=F64) * 0.1,
        'mlp.2.weight': torch.randn(W, 4 * W, generator=g, dtype=F64) / math.sqrt(4 * W),
        'mlp.2.bias': torch.randn(W, generator=g, dtype=F64) * 0.1,
    })
    if timed:
        p['ada.1.weight'] = torch.randn(6 * W, W, generator=g, dtype=F64) * 0.1
        p['ada.1.bias'] = torch.randn(6 * W, generator=g, dtype=F64) * 0.1
    return p


def test_block_gates_and_residuals():
    B, N, W, H = 2, 5, 24, 2
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, N, W, generator=g, dtype=F64)
    pos = torch.rand(B, N, 3, generator=g) * 8
    t = torch.randn(B, W, generator=g, dtype=F64)
    p = _block_params(W, 6, timed=True)
    # zero AdaLN projection: both gates are 0 and the block is the identity
    q = dict(p, **{'ada.1.weight': torch.zeros(6 * W, W, dtype=F64), 'ada.1.bias': torch.zeros(6 * W, dtype=F64)})
    assert torch.equal(O.block(x, t, pos, q, H), x)
    # gates 1, shifts and scales 0, MLP zero except its output bias: x1 = x + attn(LN(x)), out = x1 + bias
    bias = torch.zeros(6 * W, dtype=F64)
    bias[2 * W:3 * W] = 1
    bias[5 * W:] = 1
    q = dict(p, **{'ada.1.weight': torch.zeros(6 * W, W, dtype=F64), 'ada.1.bias': bias,
                   'mlp.0.weight': torch.zeros(4 * W, W, dtype=F64), 'mlp.0.bias': torch.zeros(4 * W, dtype=F64),
                   'mlp.2.weight': torch.zeros(W, 4 * W, dtype=F64)})
    x1 = x + O.rotary_attention(O.layer_norm(x, 1e-6), pos, q, H)
    assert torch.allclose(O.block(x, t, pos, q, H), x1 + q['mlp.2.bias'], rtol=1e-12, atol=1e-12)
    # the affine block with unit LayerNorms and a zero attention projection is x + MLP(LN(x))
    a = _block_params(W, 7, timed=False)
    a.update({'attn.proj.weight': torch.zeros(W, W, dtype=F64), 'attn.proj.bias': torch.zeros(W, dtype=F64)})
    want = x + O.mlp(O.layer_norm(x, 1e-6), a)
    assert torch.allclose(O.block(x, None, pos, a, H), want, rtol=1e-12, atol=1e-12)


def test_patch_embed_equals_the_one_hot_conv():
    """The gather form against torch's Conv3d of the one-hot tokens (a library routine), in float64."""
    g = torch.Generator().manual_seed(8)
    B, Y, Z, X, p, C, W = 2, 8, 4, 8, 4, 6, 5
    tokens = torch.randint(0, C + 1, (B, Y, Z, X), generator=g)
    weight = torch.randn(W, C + 1, p, p, p, generator=g, dtype=F64)
    bias = torch.randn(W, generator=g, dtype=F64)
    onehot = torch.zeros(B, C + 1, Y, Z, X, dtype=F64).scatter_(1, tokens[:, None], 1.0)
    want = torch.nn.functional.conv3d(onehot, weight, bias, stride=p).flatten(2).transpose(1, 2)
    assert torch.allclose(O.patch_embed(tokens, weight, bias, p), want, rtol=1e-12, atol=1e-12)


def test_step_forward_with_identity_blocks_is_the_head_of_the_embedding():
    """Every block's AdaLN projection zero (gates 0: blocks are identities) and the zero projections zero: the
    step's output is class_head(modulate(LN(patchify + height embedding), final shift, gain))."""
    from streamvoxel_amd import synth
    model = synth.StepModel(classes=5, voxel_shape=(8, 4, 4), patch=4, width=48, depth=2, heads=1,
                            control_width=24, control_depth=1, seed=2)
    params = {k: v.double() for k, v in model.state_dict().items()}
    for k in list(params):
        if '.ada.1.' in k or k.startswith('zero.'):
            params[k] = torch.zeros_like(params[k])
    g = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, 6, (2, 8, 4, 4), generator=g)
    t = torch.tensor([0.1, 0.9])
    origin = torch.tensor([[0.0, -64.0, 0.0], [4.0, 0.0, 8.0]])
    group = torch.zeros(3)
    keys = [torch.randn(2, 1, 8, 24, generator=g, dtype=F64)]
    out = O.step_forward(params, tokens, t, origin, group, keys, keys, [8, 3], depth=2, heads=1, control_heads=1,
                         layer_map=model.layer_map, patch=4, y_range=(-64.0, 192.0), time_dim=256,
                         voxel_shape=(8, 4, 4))
    bb = {k[len('backbone.'):]: v for k, v in params.items() if k.startswith('backbone.')}
    centers = bb['patch_centers_xyz'][None] + origin.double()[:, None]
    y = 2 * (centers[..., 1:2] + 64) / 256 - 1
    e = O.linear(O.silu(O.linear(y, bb['y_embed.0.weight'], bb['y_embed.0.bias'])), bb['y_embed.2.weight'],
                 bb['y_embed.2.bias'])
    x = O.patch_embed(tokens, bb['target_patch.weight'], bb['target_patch.bias'], 4) + e
    bt = O.time_encoding(t, bb, 256)
    shift, gain = O.linear(O.silu(bt), bb['final_ada.1.weight'], bb['final_ada.1.bias']).chunk(2, -1)
    want = O.linear(O.modulate(O.layer_norm(x, 1e-6), shift, gain), bb['class_head.weight'], bb['class_head.bias'])
    assert torch.allclose(out, want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------------------------------- reference vectors

def _fixture_params(names, prefix, dtype):
    """The fixture's weights, drawn by name from the same fill as tests/golden/make_golden.py, in `dtype` (the dtype
    the reference module ran in) and then float64 (exact: every value is a multiple of 2^-26)."""
    import _golden
    scale = 2.0 ** -3
    return {n: torch.from_numpy(_golden.hash_fill(tuple(shape), _golden.name_seed(prefix + n), scale)).to(dtype)
            .to(F64) for n, shape in names}


def test_blocks_match_the_reference_vectors():
    """UnconditionalBlock with non-zero AdaLN shifts, scales and gates, and the affine block, against the
    reference modules' float64 outputs; a swap of shift and scale (or of the two gates) misses by far more."""
    import _golden
    meta, data = _golden.forward_meta(), _golden.forward_arrays()
    for m in meta['blocks']:
        kind, W, H, N, B = m['kind'], m['width'], m['heads'], m['tokens'], m['batch']
        params = _fixture_params(m['params'], f'block_{kind}.', F64)
        x = torch.from_numpy(_golden.hash_fill((B, N, W), _golden.name_seed(f'block_{kind}.x'), 1.0))
        t = torch.from_numpy(_golden.hash_fill((B, W), _golden.name_seed(f'block_{kind}.t'), 1.0))
        pos = torch.from_numpy(np.round(_golden.hash_fill((B, N, 3), _golden.name_seed(f'block_{kind}.pos'), 8.0) * 8) / 8)
        params['attn.rope.frequencies'] = P.rope_frequencies(W // H).double()
        want = torch.from_numpy(data[f'block_{kind}/out'])
        got = O.block(x, t if kind == 'ada' else None, pos, params, H)
        torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
        if kind == 'ada':
            w, bias = params['ada.1.weight'], params['ada.1.bias']
            for a, b in ((0, 1), (2, 5)):          # (shift1, scale1), (gate1, gate2)
                perm = list(range(6))
                perm[a], perm[b] = b, a
                swapped = dict(params, **{'ada.1.weight': w.view(6, W, W)[perm].reshape(6 * W, W),
                                          'ada.1.bias': bias.view(6, W)[perm].reshape(6 * W)})
                assert (O.block(x, t, pos, swapped, H) - want).abs().max() > 1e-3


def test_time_encoding_matches_the_reference_vectors():
    """The time-conditioned model's time encoding (sinusoidal features in fp32, then the MLP; the module ran in
    fp32): within fp32 rounding of the reference, and far from it with the sines and cosines swapped."""
    import _golden
    meta, data = _golden.forward_meta(), _golden.forward_arrays()
    m = meta['time']
    params = _fixture_params(m['params'], 'time.', torch.float32)
    want = torch.from_numpy(data['time/out'])
    got = O.time_encoding(torch.tensor(m['t']), params, m['time_dim'])
    err = (got - want).abs().max().item()
    assert err <= 2e-6 * max(1.0, want.abs().max().item()), err
    w = params['time_mlp.0.weight']
    half = w.shape[1] // 2
    swapped = dict(params, **{'time_mlp.0.weight': torch.cat((w[:, half:], w[:, :half]), 1)})
    assert (O.time_encoding(torch.tensor(m['t']), swapped, m['time_dim']) - want).abs().max() > 1e-3


def _step_inputs(m):
    import _golden
    pre = f"step_{m['variant']}."
    dt = torch.float64 if m['dtype'] == 'float64' else torch.float32
    hf = lambda shape, name, scale: torch.from_numpy(_golden.hash_fill(shape, _golden.name_seed(pre + name), scale))
    u = _golden.hash_fill((1, *m['voxel_shape']), _golden.name_seed(pre + 'tokens'), 1.0)
    tokens = torch.from_numpy(np.minimum(np.floor((u + 1.0) * 2.0), 3).astype(np.int64))
    H, cw = m['control_heads'], m['control_width']
    D = cw // H
    prefix = [(hf((1, H, m['prefix'], D), f'pk{j}', 1.0), hf((1, H, m['prefix'], D), f'pv{j}', 1.0))
              for j in range(len(m['layer_map']))]
    local = hf((1, m['local'], cw), 'local', 1.0)
    lpos = torch.round(hf((1, m['local'], 3), 'local_pos', 16.0) * 8) / 8
    return tokens, prefix, local, lpos, dt


def _oracle_step(m, params, tokens, prefix, local, lpos, dt):
    """The step oracle fed the reference forward's condition: per cross layer, prefix K / V followed by the local
    K / V (the layer's key_value projection of `local`, K rotated at the local positions)."""
    H, cw = m['control_heads'], m['control_width']
    D = cw // H
    freq = P.rope_frequencies(D).to(dt)
    keys, values = [], []
    for j in range(len(m['layer_map'])):
        kv = O.linear(local, params[f'cross.{j}.key_value.weight'], params[f'cross.{j}.key_value.bias'])
        kv = kv.reshape(1, m['local'], 2, H, D)
        k = P.axial_rope(kv[:, :, 0].transpose(1, 2).contiguous(), lpos.to(dt), freq)
        keys.append(torch.cat((prefix[j][0], k), 2))
        values.append(torch.cat((prefix[j][1], kv[:, :, 1].transpose(1, 2)), 2))
    return O.step_forward(params, tokens, torch.tensor(m['timestep']), torch.tensor(m['origin'], dtype=F64),
                          torch.tensor(m['group_origin'], dtype=F64), keys, values, [m['prefix'] + m['local']],
                          depth=m['depth'], heads=m['heads'], control_heads=H,
                          layer_map={int(k): v for k, v in m['layer_map'].items()}, patch=m['patch'],
                          y_range=tuple(m['y_range']), time_dim=m['time_dim'], voxel_shape=tuple(m['voxel_shape']),
                          timed=m['variant'] != 'affine', time_free=m['variant'] == 'time_free')


def test_step_forward_matches_the_reference_vectors():
    """One step of the tiny CompactStreamingControlNet (affine, time-free and time-conditioned variants, every zero
    projection non-zero so the control -> cross attention -> injection path counts) against the reference
    forward's logits: float64 variants to 1e-10, the fp32 one to its rounding. Dropping the injections misses."""
    import _golden
    from oracle import patches as PT
    meta, data = _golden.forward_meta(), _golden.forward_arrays()
    for m in meta['step']:
        tokens, prefix, local, lpos, dt = _step_inputs(m)
        params = _fixture_params(m['params'], f"step_{m['variant']}.", dt)
        params['backbone.patch_centers_xyz'] = torch.from_numpy(data[f"step_{m['variant']}/patch_centers_xyz"])
        for j in range(len(m['layer_map'])):
            params[f'cross.{j}.rope.frequencies'] = P.rope_frequencies(m['control_width'] // m['heads']).to(dt)
        for i in range(m['depth']):
            params[f'backbone.blocks.{i}.attn.rope.frequencies'] = P.rope_frequencies(m['width'] // m['heads']).to(dt)
        for j in range(len(m['layer_map'])):
            params[f'control.blocks.{j}.attn.rope.frequencies'] = P.rope_frequencies(
                m['control_width'] // m['heads']).to(dt)
        rows = _oracle_step(m, params, tokens, prefix, local, lpos, dt)
        got = PT.to_class_major(rows.numpy(), tuple(m['voxel_shape']), m['patch'], m['classes'])
        want = data[f"step_{m['variant']}/out"]
        scale = np.abs(want).max()
        tol = 1e-10 if m['dtype'] == 'float64' else 1e-4
        err = np.abs(got - want).max()
        assert err <= tol * scale, (m['variant'], err, scale)
        cut = dict(params, **{k: torch.zeros_like(v) for k, v in params.items() if k.startswith('zero.')})
        rows = _oracle_step(m, cut, tokens, prefix, local, lpos, dt)
        missed = np.abs(PT.to_class_major(rows.numpy(), tuple(m['voxel_shape']), m['patch'], m['classes']) - want).max()
        assert missed > 100 * tol * scale, (m['variant'], missed)
