"""GPU parity at the shapes of the five workload configurations (through the C ABI).

* single column, fp32 inputs: one cross-attention layer (12 x 64 heads, 1024 queries, 9744 keys) against float64
  on the fp32 inputs; the EASE select of a fresh window (k = 2621, 4^3 blocks) in its closed form and bit-exact to
  the oracle given the kernel's scores;
* 8-slot step: packed cu_seqlens and padded layouts give the same bits;
* 12-layer cached context in one HIP graph (attention x 12 + select), replayed with fresh queries and logits, every
  replay equal to the eager kernels and spot-checked against float64;
* 64-slot e4m3 stress: 16 x 64 heads, cache written by svhip_kv_write, spot-checked against float64 on the
  dequantised K/V and batch-invariant; select over [64 x 65536, 256] fp32 logits.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import sampling as S

pytestmark = pytest.mark.gpu

SHAPE, CLASSES, BLOCK = (256, 16, 16), 256, 4
N = 65536


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _check(got, ref, atol, rtol):
    err = (got.double().cpu() - ref).abs().max().item()
    assert err <= atol, err
    assert err / ref.abs().max().item() <= rtol, (err, ref.abs().max().item())


def _fresh_select(dev, logits, batch, k, seed):
    """EaseSelect of `batch` fresh windows (nothing committed or deferred) over voxel-major logits; returns the
    selection state, chosen [B, N] (host) and the kernel's scores (host)."""
    from streamvoxel_amd.stream.step import EaseSelect
    sel = EaseSelect(batch, SHAPE, CLASSES, BLOCK, dev)
    orders = [torch.randperm(N // BLOCK ** 3, generator=torch.Generator().manual_seed(seed + b)) for b in range(batch)]
    for b in range(batch):
        sel.bind_window(b, orders[b])
        sel.set_step(b, k, 0, k / N)
    sel.run(logits, keep_scores=True)
    torch.cuda.synchronize()
    assert not bool(sel.bad.any())
    return sel, [o.numpy() for o in orders], sel.chosen.cpu().numpy(), sel.scores.cpu().numpy()


def test_single_column_fp32_attention_and_fresh_select(dev):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.attention import attention
    _case('single column: attention 12x64, Q 1024, 9744 keys, fp32 inputs and fp32 arithmetic')
    g = torch.Generator().manual_seed(2024)
    q = torch.randn(1, 12, 1024, 64, generator=g) / 8
    k = torch.randn(1, 12, 9744, 64, generator=g) / 8
    v = torch.randn(1, 12, 9744, 64, generator=g) / 8
    lt = torch.tensor([9744], dtype=torch.int32, device=dev)
    ref = A.cross_attention(q, k, v, [9744])
    out32 = attention(q.to(dev), k.to(dev), v.to(dev), lengths=lt)       # the configuration's fp32
    torch.cuda.synchronize()
    assert out32.dtype == torch.float32
    _check(out32, ref, 2e-5, 1e-4)
    # The same column through the bf16 kernel (operands rounded to bf16) holds the bf16 bar.
    out = attention(q.to(dev).bfloat16(), k.to(dev).bfloat16(), v.to(dev).bfloat16(), lengths=lt)
    torch.cuda.synchronize()
    _check(out, ref, 2e-2, 1e-2)

    _case('single column: fresh EASE select, k = 2621, 4^3 blocks')
    logits = synth.bimodal_logits(N, CLASSES, 0.7, seed=7, device=dev)
    k_sel = N // 25
    sel, orders, chosen, scores = _fresh_select(dev, logits, 1, k_sel, 77)
    assert int(chosen.sum()) == k_sel == 2621
    # Closed form: every 4^3 block gets floor(2621 / 1024) = 2, and the 573 blocks first in the permutation one more.
    pos = S.order_to_pos(orders[0])
    per_block = S.block_view(chosen[0].reshape(SHAPE), BLOCK).sum(1)
    assert np.array_equal(per_block, 2 + (pos < 2621 - 2048))
    want = S.block_quota_select(scores[0].reshape(SHAPE), np.ones(SHAPE, bool), k_sel, BLOCK, orders[0],
                                k_sel / N, S.block_view(np.ones(SHAPE, bool), BLOCK).sum(1))
    assert np.array_equal(chosen[0].reshape(SHAPE), want)


def test_eight_slot_packed_equals_padded(dev):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.attention import attention
    lengths = synth.kv_lengths(8, 31)
    _case(f'8-slot packed vs padded, lengths={lengths}')
    g = torch.Generator(device=dev).manual_seed(31)
    B, H, Q, D, kcap = 8, 12, 1024, 64, 9792
    q = (torch.randn(B, H, Q, D, device=dev, generator=g) / 8).bfloat16()
    k = (torch.randn(B, H, kcap, D, device=dev, generator=g) / 8).bfloat16()
    v = (torch.randn(B, H, kcap, D, device=dev, generator=g) / 8).bfloat16()
    padded = attention(q, k, v, lengths=torch.tensor(lengths, dtype=torch.int32, device=dev))
    kp = torch.cat([k[b, :, :L] for b, L in enumerate(lengths)], 1)       # [H, sum L, D]
    vp = torch.cat([v[b, :, :L] for b, L in enumerate(lengths)], 1)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32, device=dev)
    packed = attention(q, kp, vp, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert torch.equal(packed, padded)


def test_twelve_layer_context_graph_replays(dev):
    """One graph = 12 attention layers over the cached context + the EASE select; three replays with new queries
    and logits copied into the static inputs between them (eager work in between), each equal to the eager
    kernels on the same inputs."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.step import CachedContext, EaseSelect
    layers, B, H, Q, D = 12, 8, 12, 1024, 64
    lengths = synth.kv_lengths(B, 5)
    _case(f'12-layer graph, lengths={lengths}')
    g = torch.Generator(device=dev).manual_seed(5)
    ctx = CachedContext(layers, B, H, D, synth.MAX_KEYS, dev)
    for layer in range(layers):
        for b, L in enumerate(lengths):
            ctx.write(layer, b, (torch.randn(H, L, D, device=dev, generator=g) / 8).bfloat16(),
                      (torch.randn(H, L, D, device=dev, generator=g) / 8).bfloat16())
    qbuf = [torch.empty(B, Q, H, D, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    obuf = [torch.empty(B, Q, H, D, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    sel = EaseSelect(B, SHAPE, CLASSES, BLOCK, dev)
    for b in range(B):
        sel.bind_window(b, torch.randperm(N // 64, generator=torch.Generator().manual_seed(b)))
        sel.set_step(b, 1000 + b, 0, (1000 + b) / N)
    logits = torch.empty(B * N, CLASSES, device=dev)
    # the captured step reads the step's scalars from table rows in place (scalars=), the eager one from the
    # selection's own buffers: the same values, so the same bits
    tables = (sel.k.clone(), sel.committed.clone(), sel.frac.clone())

    def step(scalars=None):
        for layer in range(layers):
            ctx.attend(layer, qbuf[layer].transpose(1, 2), out=obuf[layer].transpose(1, 2))
        sel.run(logits, scalars=scalars)

    def fill(seed):
        gg = torch.Generator(device=dev).manual_seed(seed)
        for t in qbuf:
            t.copy_((torch.randn(t.shape, device=dev, generator=gg) / 8).bfloat16())
        synth.bimodal_logits_(logits, 0.8, generator=gg)

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(tables)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(tables)
    for replay in range(3):
        fill(100 + replay)
        graph.replay()
        torch.cuda.synchronize()
        got_o = [o.clone() for o in obuf]
        got_c = sel.chosen.clone()
        step()                                            # eager, same inputs
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(got_o[layer], obuf[layer]), (replay, layer)
        assert torch.equal(got_c, sel.chosen), replay
        assert not bool(sel.bad.any())
    with pytest.raises(ValueError, match='frac'):
        sel.run(logits, scalars=(tables[0], tables[1], tables[2].float()))
    with pytest.raises(ValueError, match='k must'):
        sel.run(logits, scalars=(tables[0][:B - 1], tables[1], tables[2]))
    # Spot check of the last replay against float64: two windows, two heads, every 16th query, layers 0 and 11.
    for layer in (0, layers - 1):
        for b in (0, 5):
            qh = qbuf[layer][b:b + 1, ::16, [1, 7]].transpose(1, 2).cpu()
            kh = ctx.k[layer][b:b + 1, [1, 7]].cpu()
            vh = ctx.vt[layer][b:b + 1, [1, 7]].cpu().transpose(2, 3)
            ref = A.cross_attention(qh, kh, vh, [lengths[b]])
            _check(obuf[layer][b:b + 1, ::16, [1, 7]].transpose(1, 2), ref, 2e-2, 1e-2)


def test_sixty_four_slot_e4m3_stress(dev):
    """64 windows, 16 x 64 heads (hidden 1024), K/V projected from seeded context tokens (as the bench's stress)
    and written as an e4m3 cache by svhip_kv_write. The default form (bf16 softmax weights over the exactly
    decoded cache) and the opt-in fp8 second product both hold 5e-2 against float64 attention over the ORIGINAL
    bf16 K/V (quantisation included), and the kernel's own arithmetic holds it against float64 over the
    dequantised cache."""
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.attention import attention
    from streamvoxel_amd.stream.step import CachedContext
    B, H, Q, D = 64, 16, 1024, 64
    W = H * D
    lengths = synth.kv_lengths(B, 64)
    _case(f'64-slot e4m3: sum L = {sum(lengths)}')
    g = torch.Generator(device=dev).manual_seed(64)
    ctx = CachedContext(1, B, H, D, synth.MAX_KEYS, dev, kv_dtype='fp8')
    assert ctx.p_dtype == 'bf16'
    proj = torch.randn(W, 2 * W, device=dev, generator=g) / math.sqrt(W)
    raw = {}
    for b, L in enumerate(lengths):
        kv = (torch.randn(L, W, device=dev, generator=g) @ proj).reshape(L, 2, H, D).permute(1, 2, 0, 3)
        kb, vb = kv[0].bfloat16(), kv[1].bfloat16()
        ctx.write(0, b, kb, vb)
        if b in (0, 17, 63):
            raw[b] = (kb, vb)
    q = (torch.randn(B, Q, H, D, device=dev, generator=g) / 8).bfloat16()
    out = ctx.attend(0, q.transpose(1, 2))
    out_pfp8 = attention(q.transpose(1, 2), ctx.k[0], ctx.vt[0].transpose(2, 3), lengths=ctx.lengths,
                         k_scale=ctx.k_scale[0], v_scale=ctx.v_scale[0], p_dtype='e4m3')
    torch.cuda.synchronize()
    for b, (kb, vb) in raw.items():
        # Against the unquantised keys and values: float64 attention over the bf16 K/V the cache was written from.
        qh = q[b, ::16, [3, 12]].transpose(0, 1).cpu()
        ref = A.cross_attention(qh[None], kb[[3, 12]][None].cpu(), vb[[3, 12]][None].cpu(), [lengths[b]])
        for name, o in (('default', out), ('pfp8', out_pfp8)):
            err = (o[b:b + 1, [3, 12], ::16].double().cpu() - ref).abs().max().item()
            print(f'[gpu-case] 64-slot e4m3 {name} window {b}: |kernel - f64 over the original K/V| {err:.2e} '
                  f'(max |ref| {ref.abs().max().item():.2e})', flush=True)
            # 5e-2 absolute (the fp8 bar); the default form also within 5e-2 of the output's own scale (measured
            # 2-2.5 %; the fp8 second product about twice that)
            _check(o[b:b + 1, [3, 12], ::16], ref, 5e-2, 5e-2 if name == 'default' else 1.0)
    for b in raw:
        # Dequantised cache = what the kernel multiplies; float64 attention over it, 2 heads, every 16th query.
        L = lengths[b]
        kd = A.dequant_e4m3(ctx.k[0][b, [3, 12], :L].view(torch.uint8).cpu(), 1.0) * \
            ctx.k_scale[0][b, [3, 12]].cpu().double()[:, None, None]
        vd = A.dequant_e4m3(ctx.vt[0][b, [3, 12], :, :L].view(torch.uint8).cpu(), 1.0).transpose(1, 2) * \
            ctx.v_scale[0][b, [3, 12]].cpu().double()[:, None, None]
        qh = q[b, ::16, [3, 12]].transpose(0, 1).cpu()
        ref = A.cross_attention(qh[None], kd[None], vd[None], [L])
        _check(out[b:b + 1, [3, 12], ::16], ref, 5e-2, 5e-2)
    # Batch invariance: window 17 alone, written and attended by itself, gives the same bits.
    sub = CachedContext(1, 1, H, D, synth.MAX_KEYS, dev, kv_dtype='fp8')
    kb, vb = raw[17]
    sub.write(0, 0, kb, vb)
    one = sub.attend(0, q[17:18].transpose(1, 2))
    torch.cuda.synchronize()
    assert torch.equal(one, out[17:18])

    _case('64-slot select over [64 x 65536, 256] fp32')
    logits = torch.empty(B * N, CLASSES, device=dev)
    synth.bimodal_logits_(logits, 0.7, generator=torch.Generator(device=dev).manual_seed(65))
    sel, orders, chosen, scores = _fresh_select(dev, logits, B, 2621, 900)
    assert np.all(chosen.reshape(B, -1).sum(1) == 2621)
    ones = np.ones(SHAPE, bool)
    for b in (0, 31, 63):
        want = S.block_quota_select(scores[b].reshape(SHAPE), ones, 2621, BLOCK, orders[b], 2621 / N,
                                    S.block_view(ones, BLOCK).sum(1))
        assert np.array_equal(chosen[b].reshape(SHAPE), want), b
