"""GPU parity of the transformer-block path (streamvoxel_amd.stream.backbone): the fused qkv producer against the
golden-pinned AxialRoPE kernel and an exact transpose, the fused LayerNorm + AdaLN modulation against the float64
oracle, and whole blocks (AdaLN at the 384- and 768-wide shapes, affine) against the float64 oracle block.

Tolerances: LayerNorm output within bf16 rounding (2^-8 relative, plus the rounding of 1 + scale to bf16 that the
reference's bf16 tensors make); a whole block within 3e-2 of max |reference| (max-abs) and 4e-3 of mean |reference|
(mean-abs), against float64 on the same bf16 weights and inputs."""
import pytest
import torch

from oracle import backbone as O

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


@pytest.mark.parametrize('B,N,W,H', [(2, 1024, 384, 8), (2, 200, 768, 8), (1, 77, 480, 5)])
def test_qkv_rope_equals_axial_rope_and_transpose(dev, B, N, W, H):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.backbone import qkv_rope
    from streamvoxel_amd.stream.producer import axial_rope, rope_frequencies
    _case(f'qkv_rope B={B} N={N} W={W} H={H}')
    D = W // H
    g = torch.Generator().manual_seed(N + W)
    qkv = torch.randn(B, N, 3 * W, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.rand(B, N, 3, generator=g).to(dev) * 64
    if N == 1024:
        pos = synth.patch_positions().to(dev)[None].expand(B, -1, -1)
    freq = rope_frequencies(D, device=dev)
    view = qkv.clone().view(B, N, 3, H, D)
    want_q = axial_rope(view[:, :, 0].transpose(1, 2), pos, freq)
    want_k = axial_rope(view[:, :, 1].transpose(1, 2), pos, freq)
    want_vt = view[:, :, 2].permute(0, 2, 3, 1)
    q, k, vt = qkv_rope(qkv, pos, freq, H)
    torch.cuda.synchronize()
    assert q.data_ptr() == qkv.data_ptr()                       # rotated in place
    assert torch.equal(q, want_q) and torch.equal(k, want_k)
    assert torch.equal(vt[..., :N], want_vt)


@pytest.mark.parametrize('W,affine,modulated', [(384, False, True), (768, False, True), (768, True, False),
                                                (1280, True, True), (200, False, False)])
def test_layer_norm_against_oracle(dev, W, affine, modulated):
    from streamvoxel_amd.stream.backbone import layer_norm
    _case(f'layer_norm W={W} affine={affine} modulated={modulated}')
    B, N = 3, 333
    g = torch.Generator().manual_seed(W)
    x = (torch.randn(B, N, W, generator=g) * 2 + 0.5).to(torch.bfloat16)
    norm = torch.nn.LayerNorm(W, elementwise_affine=affine, eps=1e-6)
    if affine:
        with torch.no_grad():
            norm.weight.copy_(1 + torch.randn(W, generator=g) * 0.2)
            norm.bias.copy_(torch.randn(W, generator=g) * 0.2)
    shift = scale = None
    if modulated:
        ada = (torch.randn(B, 6 * W, generator=g) * 0.3).to(torch.bfloat16)
        shift, scale = ada[:, :W], ada[:, W:2 * W]                # strided [B, W] views, as chunk() gives
    w = b = None
    if affine:
        w, b = norm.weight.detach().clone(), norm.bias.detach().clone()
    y = layer_norm(x.to(dev), norm.to(dev), None if shift is None else shift.to(dev),
                   None if scale is None else scale.to(dev))
    torch.cuda.synchronize()
    ref = O.layer_norm(x, 1e-6, w, b)
    bound = 2.0 ** -8 * ref.abs()
    if modulated:
        onep = (1 + scale.double()).to(torch.bfloat16).double()   # the reference rounds 1 + scale to bf16
        ref = ref * onep[:, None] + shift.double()[:, None]
        bound = 2.0 ** -8 * ref.abs() + 2.0 ** -8 * (ref - shift.double()[:, None]).abs()
    err = (y.cpu().double() - ref).abs()
    assert bool((err <= bound + 1e-5).all()), float((err - bound).max())


@pytest.mark.parametrize('W,gated,normed', [(768, True, True), (384, True, False), (384, False, True)])
def test_residual_norm(dev, W, gated, normed):
    """r = x + g * a must equal torch's bf16 `x + g[:, None] * a` bit for bit (the reference's roundings); y as the
    LayerNorm test bounds it."""
    from streamvoxel_amd.stream.backbone import residual_norm
    _case(f'residual_norm W={W} gated={gated} normed={normed}')
    B, N = 3, 257
    g = torch.Generator().manual_seed(W + 7)
    x = torch.randn(B, N, W, generator=g).to(torch.bfloat16).to(dev)
    a = (torch.randn(B, N, W, generator=g) * 3).to(torch.bfloat16).to(dev)
    ada = (torch.randn(B, 6 * W, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    s2, c2, g2 = ada[:, 3 * W:4 * W], ada[:, 4 * W:5 * W], ada[:, 5 * W:]
    norm = torch.nn.LayerNorm(W, elementwise_affine=False, eps=1e-6)
    out = residual_norm(x, a, g2 if gated else None, norm if normed else None, s2 if normed else None,
                        c2 if normed else None)
    want = x + g2[:, None] * a if gated else x + a
    torch.cuda.synchronize()
    r, y = out if normed else (out, None)
    assert torch.equal(r, want)
    if normed:
        ref = O.layer_norm(r.cpu(), 1e-6)
        onep = (1 + c2.cpu().double()).to(torch.bfloat16).double()
        sh = s2.cpu().double()
        ref = ref * onep[:, None] + sh[:, None]
        bound = 2.0 ** -8 * ref.abs() + 2.0 ** -8 * (ref - sh[:, None]).abs()
        err = (y.cpu().double() - ref).abs()
        assert bool((err <= bound + 1e-5).all()), float((err - bound).max())


def _check_block(out, ref):
    out = out.float().cpu().double()
    err = (out - ref).abs()
    assert float(err.max()) <= 3e-2 * float(ref.abs().max()), (float(err.max()), float(ref.abs().max()))
    assert float(err.mean()) <= 4e-3 * float(ref.abs().mean()), (float(err.mean()), float(ref.abs().mean()))


@pytest.mark.parametrize('W,H,timed', [(384, 8, True), (768, 8, True), (384, 8, False)])
def test_block_against_oracle(dev, W, H, timed):
    from streamvoxel_amd import synth
    from streamvoxel_amd.stream.backbone import run_block
    _case(f'block W={W} H={H} timed={timed}')
    B = 2
    block = synth.BlockWeights(W, H, timed=timed, seed=W)
    for p in block.parameters():                                 # bf16 weights; the rope buffer stays fp32
        p.data = p.data.to(torch.bfloat16)
    g = torch.Generator().manual_seed(W + 1)
    x = torch.randn(B, 1024, W, generator=g).to(torch.bfloat16)
    t = (torch.randn(B, W, generator=g) * 2).to(torch.bfloat16) if timed else None
    pos = synth.patch_positions()[None].expand(B, -1, -1).contiguous()
    with torch.no_grad():
        bd = block.to(dev)
        out = run_block(bd, x.to(dev), None if t is None else t.to(dev), pos.to(dev))
        torch.cuda.synchronize()
    params = {k: v.cpu() for k, v in block.state_dict().items()}
    ref = O.block(x, t, pos, params, H)
    _check_block(out, ref)


def test_in_place_forms(dev):
    """The forms the C ABI documents as allowed: the residual written over x (svhip_residual_norm with r = x) and
    LayerNorm written over its input; both equal the out-of-place results bit for bit."""
    from streamvoxel_amd import _lib
    from streamvoxel_amd.stream.backbone import layer_norm, residual_norm
    _case('in-place residual / layer_norm')
    B, N, W = 2, 130, 768
    g = torch.Generator().manual_seed(41)
    x = torch.randn(B, N, W, generator=g).to(torch.bfloat16).to(dev)
    a = torch.randn(B, N, W, generator=g).to(torch.bfloat16).to(dev)
    ada = (torch.randn(B, 3 * W, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    gate, shift, scale = ada[:, :W], ada[:, W:2 * W], ada[:, 2 * W:]
    norm = torch.nn.LayerNorm(W, elementwise_affine=False, eps=1e-6)
    r_ref, y_ref = residual_norm(x, a, gate, norm, shift, scale)
    xi = x.clone()
    lib = _lib.load()
    rc = lib.svhip_residual_norm(_lib.ptr(xi), _lib.ptr(a), _lib.ptr(gate), gate.stride(0), _lib.ptr(xi), None, None,
                                 None, None, None, 0, B, N, W, xi.stride(0), xi.stride(1), a.stride(0), a.stride(1),
                                 xi.stride(0), xi.stride(1), 0, 0, 1e-6, _lib.stream_of(xi))
    assert rc == 0, lib.svhip_last_error()
    yi = r_ref.clone()
    layer_norm(yi, norm, shift, scale, out=yi)
    torch.cuda.synchronize()
    assert torch.equal(xi, r_ref)
    assert torch.equal(yi, y_ref)
