"""GPU parity of the generation step's forward (streamvoxel_amd.stream.forward): the gather patchify against the
float64 oracle (and bit for bit against torch's embedding bag, the reference's form), and a whole step of a small
streaming ControlNet (3 backbone blocks, 2 control blocks with cross attention over a cached context) against the
float64 oracle step.

Tolerances: patchify within bf16 rounding of the fp32 sum plus the bias add (2^-8 relative of each); the step's
class-head rows within 4e-2 of max |reference| (max-abs) and 1e-2 of mean |reference| (mean-abs): every stage of
the step adds bf16 roundings (measured against float64, as mean relative errors: patchify 0.2%, time encoding
0.4%, each block about 0.05% more, the class head alone on exact inputs 0.2%; the whole step about 0.6%)."""
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


@pytest.mark.parametrize('W,shape,C,p', [(768, (64, 16, 16), 304, 4), (384, (32, 8, 8), 20, 4), (200, (8, 4, 4), 3, 4),
                                        (256, (16, 8, 8), 12, 2)])
def test_gather_patch(dev, W, shape, C, p):
    from streamvoxel_amd.stream.forward import GatherPatch
    _case(f'gather patch W={W} shape={shape} C={C} p={p}')
    g = torch.Generator().manual_seed(W)
    conv = torch.nn.Conv3d(C + 1, W, p, stride=p)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * 0.3)
        conv.bias.copy_(torch.randn(W, generator=g))
    conv = conv.to(torch.bfloat16)
    B = 2
    tokens = torch.randint(0, C + 1, (B, *shape), generator=g)
    tokens[0, :8] = C                                             # mask tokens in bulk, as early steps have
    gp = GatherPatch(conv.to(dev))
    out = gp(tokens.to(dev))
    # the reference's form: patch_offsets + embedding_bag(mode='sum') + bias, in bf16
    Y, Z, X = shape
    cells = tokens.reshape(B, Y // p, p, Z // p, p, X // p, p).permute(0, 1, 3, 5, 2, 4, 6).reshape(-1, p ** 3)
    index = (cells * p ** 3 + torch.arange(p ** 3)).to(dev)
    ref_bag = (torch.nn.functional.embedding_bag(index, gp.table, mode='sum') + gp.bias).reshape(B, -1, W)
    torch.cuda.synchronize()
    assert int(gp.bad.item()) == 0
    assert torch.equal(out, ref_bag)
    sums = O.patch_embed(tokens, conv.weight.cpu(), None, p)
    ref = sums + conv.bias.cpu().double()
    bound = 2.0 ** -8 * (sums.abs() + ref.abs()) + 1e-6
    assert bool(((out.cpu().double() - ref).abs() <= bound).all())


def test_gather_patch_flags_tokens_out_of_range(dev):
    from streamvoxel_amd.stream.forward import GatherPatch
    _case('gather patch out-of-range token')
    conv = torch.nn.Conv3d(5, 64, 4, stride=4).to(torch.bfloat16).to(dev)
    gp = GatherPatch(conv)
    tokens = torch.zeros(1, 8, 4, 4, dtype=torch.int64, device=dev)
    gp(tokens)
    torch.cuda.synchronize()
    assert int(gp.bad.item()) == 0
    tokens[0, 3, 2, 1] = 5
    gp(tokens)
    torch.cuda.synchronize()
    assert int(gp.bad.item()) != 0


def _small_model(dev):
    from streamvoxel_amd import synth
    model = synth.StepModel(classes=16, voxel_shape=(32, 8, 8), patch=4, width=192, depth=3, heads=4,
                            control_width=96, control_depth=2, seed=5)
    for p in model.parameters():                                  # bf16 weights; buffers stay fp32
        p.data = p.data.to(torch.bfloat16)
    return model.to(dev)


def test_step_forward_against_oracle(dev):
    from streamvoxel_amd.stream.forward import StepForward
    from streamvoxel_amd.stream.step import CachedContext
    _case('step forward small model')
    model = _small_model(dev)
    n, kcap = 2, 192
    lengths = [150, 37]
    H, D = 4, 24                                                  # control width 96 over the model's 4 heads
    ctx = CachedContext(2, n, H, D, kcap, dev)
    g = torch.Generator().manual_seed(11)
    keys, values = [], []
    for j in range(2):
        for b in range(n):
            k = (torch.randn(H, lengths[b], D, generator=g) / 2).to(torch.bfloat16)
            v = torch.randn(H, lengths[b], D, generator=g).to(torch.bfloat16)
            ctx.write(j, b, k.to(dev), v.to(dev))
        keys.append(ctx.k[j].cpu())
        values.append(ctx.vt[j].cpu().transpose(2, 3))
    tokens = torch.randint(0, 17, (n, 32, 8, 8), generator=g)
    timestep = torch.tensor([0.25, 0.75])
    origin = torch.tensor([[16.0, -64.0, 32.0], [0.0, -64.0, 48.0]])
    group = torch.tensor([0.0, -64.0, 16.0])
    step = StepForward(model, ctx)
    out = step(tokens.to(dev), timestep.to(dev), origin.to(dev), group.to(dev))
    torch.cuda.synchronize()
    params = {k: v.cpu() for k, v in model.state_dict().items()}
    ref = O.step_forward(params, tokens, timestep, origin, group, keys, values, lengths, depth=3, heads=4,
                         control_heads=H, layer_map=model.layer_map, patch=4, y_range=(-64.0, 192.0), time_dim=256,
                         voxel_shape=(32, 8, 8))
    got = out.patches.float().cpu().double()
    err = (got - ref).abs()
    assert float(err.max()) <= 4e-2 * float(ref.abs().max()), (float(err.max()), float(ref.abs().max()))
    assert float(err.mean()) <= 1e-2 * float(ref.abs().mean()), (float(err.mean()), float(ref.abs().mean()))


def test_step_forward_graph_replays_equal_eager(dev):
    """The step forward captured in one graph and replayed three times with new tokens, timesteps and origins written
    into its static inputs (eager work and synchronisations between the replays): every replay's class-head rows
    equal the eager forward's on the same inputs bit for bit."""
    from streamvoxel_amd.stream.forward import StepForward
    from streamvoxel_amd.stream.step import CachedContext
    _case('step forward graph replays')
    model = _small_model(dev)
    n, H, D, kcap = 2, 4, 24, 192
    ctx = CachedContext(2, n, H, D, kcap, dev)
    g = torch.Generator().manual_seed(21)
    for j in range(2):
        for b, L in enumerate([120, 64]):
            ctx.write(j, b, (torch.randn(H, L, D, generator=g) / 2).to(torch.bfloat16).to(dev),
                      torch.randn(H, L, D, generator=g).to(torch.bfloat16).to(dev))
    step = StepForward(model, ctx)
    tokens = torch.zeros(n, 32, 8, 8, dtype=torch.int64, device=dev)
    timestep = torch.zeros(n, device=dev)
    origin = torch.zeros(n, 3, device=dev)
    group = torch.tensor([0.0, -64.0, 0.0], device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(tokens, timestep, origin, group)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step(tokens, timestep, origin, group)
    for r in range(3):
        tokens.copy_(torch.randint(0, 17, (n, 32, 8, 8), generator=g).to(dev))
        timestep.copy_(torch.rand(n, generator=g).to(dev))
        origin.copy_(torch.tensor([[16.0 * r, -64.0, 0.0], [0.0, -64.0, 16.0 * r]], device=dev))
        graph.replay()
        torch.cuda.synchronize()
        replayed = captured.patches.clone()
        eager = step(tokens, timestep, origin, group).patches
        torch.randn(1000, device=dev).sum()                       # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), r


@pytest.mark.parametrize('p_dtype', ['bf16', 'e4m3'])
def test_step_forward_over_an_e4m3_context(dev, p_dtype):
    """The same small step over a cached context stored as e4m3 codes with per-(window, head) scales (written by
    svhip_kv_write from the bf16 keys and values): against the float64 step on the dequantised keys and values,
    within the e4m3 bar of the attention (5e-2 of max |reference|, max-abs) and, with bf16 softmax weights, 1e-2
    of mean |reference| (2e-2 with the weights rounded to e4m3 for the fp8 matrix cores: a 2^-4 relative rounding
    that the blocks carry to the class head)."""
    from oracle import attention as A
    from streamvoxel_amd.stream.forward import StepForward
    from streamvoxel_amd.stream.step import CachedContext
    if not hasattr(torch, 'float8_e4m3fn'):
        pytest.skip('torch without float8_e4m3fn')
    _case(f'step forward e4m3 context P={p_dtype}')
    model = _small_model(dev)
    n, H, D, kcap = 2, 4, 24, 192
    lengths = [150, 37]
    ctx = CachedContext(2, n, H, D, kcap, dev, kv_dtype='fp8', p_dtype=p_dtype)
    g = torch.Generator().manual_seed(31)
    keys, values = [], []
    for j in range(2):
        for b in range(n):
            k = (torch.randn(H, lengths[b], D, generator=g) / 2).to(torch.bfloat16)
            v = torch.randn(H, lengths[b], D, generator=g).to(torch.bfloat16)
            ctx.write(j, b, k.to(dev), v.to(dev))
        ks = ctx.k_scale[j].cpu()[:, :, None, None]
        vs = ctx.v_scale[j].cpu()[:, :, None, None]
        keys.append(A.dequant_e4m3(ctx.k[j].view(torch.uint8).cpu(), ks))
        values.append(A.dequant_e4m3(ctx.vt[j].view(torch.uint8).cpu().transpose(2, 3), vs))
    tokens = torch.randint(0, 17, (n, 32, 8, 8), generator=g)
    timestep = torch.tensor([0.4, 0.6])
    origin = torch.tensor([[16.0, -64.0, 32.0], [0.0, -64.0, 48.0]])
    group = torch.tensor([0.0, -64.0, 16.0])
    out = StepForward(model, ctx)(tokens.to(dev), timestep.to(dev), origin.to(dev), group.to(dev))
    torch.cuda.synchronize()
    params = {k: v.cpu() for k, v in model.state_dict().items()}
    ref = O.step_forward(params, tokens, timestep, origin, group, keys, values, lengths, depth=3, heads=4,
                         control_heads=H, layer_map=model.layer_map, patch=4, y_range=(-64.0, 192.0), time_dim=256,
                         voxel_shape=(32, 8, 8))
    err = (out.patches.float().cpu().double() - ref).abs()
    assert float(err.max()) <= 5e-2 * float(ref.abs().max()), (float(err.max()), float(ref.abs().max()))
    mean_bar = 1e-2 if p_dtype == 'bf16' else 2e-2
    assert float(err.mean()) <= mean_bar * float(ref.abs().mean()), (float(err.mean()), float(ref.abs().mean()))
