"""The selection entry point that allocates nothing (`svhip_ease_select_noalloc`, scratch in a fixed device array of
the library) against `svhip_ease_select` with a caller workspace, through the C ABI: chosen, bad and scores
bit-identical on two calls in a row, the second with fewer and smaller windows (so it runs on the scratch the first
call left behind), and the selection bit-exact to the oracle given the kernel's own scores."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f'[gpu-case] {msg}', flush=True)


@pytest.fixture(scope='module')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no GPU')
    import streamvoxel_amd
    streamvoxel_amd.load()
    return torch.device('cuda:0')


def _state(B, shape, b, C, seed):
    """B windows mid-way: ragged deferred column tops, some committed tokens, bimodal fp32 logits [B, N, C]."""
    g = np.random.default_rng(seed)
    tg = torch.Generator().manual_seed(seed)
    Y, Z, X = shape
    N = Y * Z * X
    nb = N // b ** 3
    logits = torch.randn((B, N, C), generator=tg)
    hot = torch.rand((B, N), generator=tg) < 0.7
    cls = torch.randint(C, (B, N), generator=tg)
    logits[hot, cls[hot]] += 12.0
    tokens = np.full((B, N), C, np.int64)
    last = np.zeros((B, N), bool)
    ks, poss, fracs, nts, coms = [], [], [], [], []
    for i in range(B):
        tops = g.integers(Y // 2, Y + 1, (Z, X))
        lm = (np.arange(Y)[:, None, None] >= tops[None]).reshape(-1)
        last[i] = lm
        done = (~lm) & (g.random(N) < 0.1 * (i % 4))
        tokens[i][done] = g.integers(0, C, done.sum())
        k = max(1, N // 25 - 37 * i)
        ks.append(k)
        coms.append(int(done.sum()))
        fracs.append((coms[-1] + k) / int((~lm).sum()))
        poss.append(S.order_to_pos(g.permutation(nb)))
        nts.append(S.block_view((~lm).reshape(shape), b).sum(1))
    return logits, tokens, last, ks, poss, fracs, nts, coms


def _run(dev, B, shape, b, C, seed):
    from streamvoxel_amd import _lib
    from streamvoxel_amd.sampling.block_quota import QuotaWorkspace
    _case(f'noalloc select B={B} shape={shape} b={b} C={C} seed={seed}')
    logits, tokens, last, ks, poss, fracs, nts, coms = _state(B, shape, b, C, seed)
    N = int(np.prod(shape))
    d = lambda a, dt: torch.as_tensor(np.asarray(a), dtype=dt).to(dev)
    xd = logits.contiguous().to(dev)
    tk, ls = d(tokens, torch.int64), d(last, torch.bool)
    k_t, pos_t, frac_t = d(ks, torch.int64), d(np.stack(poss), torch.int64), d(fracs, torch.float64)
    nt_t, com_t = d(np.stack(nts), torch.int64), d(coms, torch.int64)
    lib = _lib.load()
    args = lambda chosen, bad, scores: (
        _lib.ptr(xd), _lib.SVHIP_F32, C, xd.stride(0), xd.stride(2), xd.stride(1), _lib.ptr(tk), C,
        _lib.ptr(ls.view(torch.uint8)), B, *shape, b, _lib.ptr(k_t), _lib.ptr(pos_t), _lib.ptr(frac_t),
        _lib.ptr(nt_t), _lib.ptr(com_t), _lib.ptr(chosen.view(torch.uint8)), _lib.ptr(bad.view(torch.uint8)),
        _lib.ptr(scores))
    outs = []
    for _ in range(2):
        outs.append((torch.full((B, N), True, dtype=torch.bool, device=dev),
                     torch.full((B,), True, dtype=torch.bool, device=dev),
                     torch.full((B, N), float('nan'), dtype=torch.float32, device=dev)))
    ws = QuotaWorkspace(B, shape, b, dev, fused=True)
    _lib.check(lib.svhip_ease_select(*args(*outs[0]), _lib.ptr(ws.buffer), ws.buffer.numel(), _lib.stream_of(xd)),
               'svhip_ease_select')
    _lib.check(lib.svhip_ease_select_noalloc(*args(*outs[1]), _lib.stream_of(xd)), 'svhip_ease_select_noalloc')
    torch.cuda.synchronize()
    (c0, b0, s0), (c1, b1, s1) = outs
    assert torch.equal(c0, c1)
    assert torch.equal(b0, b1)
    assert torch.equal(s0.view(torch.int32), s1.view(torch.int32))
    hs = s1.cpu().numpy()
    for i in range(B):
        selectable = (tokens[i] == C) & ~last[i]
        expect = S.quota_select_nosync(hs[i].reshape(shape), selectable.reshape(shape), ks[i], b, poss[i], fracs[i],
                                       nts[i], coms[i])
        assert np.array_equal(c1[i].cpu().numpy().reshape(shape), expect), i
        assert not bool(b1[i]), i
    return c1


def test_noalloc_select_equals_workspace_select_two_calls(dev):
    # first call: 8 windows of [256, 16, 16]; second: 3 windows of [64, 16, 16], on the scratch the first left
    _run(dev, 8, (256, 16, 16), 4, 256, seed=31)
    _run(dev, 3, (64, 16, 16), 4, 256, seed=32)
