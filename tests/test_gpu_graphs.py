"""GPU: HIP graph capture of the library's operators.

The entry points allocate nothing themselves (workspaces come from the caller, here torch's
allocator), never synchronise with the host and record no memset nodes (buffers that must start
at zero are cleared by a fill kernel), so ``torch.cuda.CUDAGraph`` can capture them as they are.
Each test captures one operator family -- the FP8 attention operator (the Q / K / V quantise pair
and the attention kernel), the FP8 linear in each recipe, the FP8 decoder block forward inside
``fp8_weight_cache``, the bf16 sliding-window attention forward, a whole training step of the block
(forward and backward) -- then replays the graph several
times with new values copied into the captured inputs, running the same operator eagerly on those
values and synchronising between the replays, and compares every replay with that eager call bit
for bit.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _seeded(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to("cuda", dtype)


def _capture(fn):
    """torch's capture recipe: warm up on a side stream (default priority), then capture."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    torch.cuda.synchronize()
    return graph, out


def _replay_and_compare(graph, out, inputs, make_inputs, eager):
    """Replay with new input values; each replay must equal the eager call on those values."""
    outs = out if isinstance(out, (list, tuple)) else [out]
    previous = None
    for i in range(REPLAYS):
        new = make_inputs(i)
        for dst, src in zip(inputs, new):
            dst.copy_(src)
        graph.replay()
        want = eager(*new)
        wants = want if isinstance(want, (list, tuple)) else [want]
        torch.cuda.synchronize()
        for got, exp in zip(outs, wants):
            assert torch.equal(got, exp), f"replay {i} differs from the eager call"
        snapshot = [o.clone() for o in outs]
        if previous is not None:           # the replay recomputed on the new values
            assert any(not torch.equal(a, b) for a, b in zip(snapshot, previous))
        previous = snapshot


@pytest.mark.parametrize("granularity", ["tensor", "head"])
def test_fp8_attention_operator_in_a_graph(granularity):
    from flower_amd.kernels import fp8_swa_attention_forward
    shape, W = (2, 4, 1000, 64), 300

    def make(i):
        return [_seeded(shape, 100 * i + s, scale=s + 1) for s in (1, 2, 3)]
    q, k, v = make(99)
    graph, out = _capture(lambda: fp8_swa_attention_forward(q, k, v, W, granularity=granularity))
    _replay_and_compare(graph, out, (q, k, v), make,
                        lambda a, b, c: fp8_swa_attention_forward(a, b, c, W, granularity=granularity))


@pytest.mark.parametrize("recipe", ["tensorwise", "rowwise", "weight_only"])
def test_fp8_linear_in_a_graph(recipe):
    from flower_amd.precision import Fp8Linear
    torch.manual_seed(0)
    lin = Fp8Linear(1024, 2048, bias=True, recipe=recipe).to("cuda", torch.bfloat16)

    def make(i):
        return [_seeded((4096, 1024), 200 + i)]
    (x,) = make(99)
    with torch.no_grad():
        graph, out = _capture(lambda: lin(x))
        _replay_and_compare(graph, out, (x,), make, lambda a: lin(a))


def test_fp8_decoder_block_in_a_graph():
    from flower_amd.block import Fp8DecoderBlock, init_block_
    from flower_amd.precision import fp8_weight_cache
    blk = Fp8DecoderBlock(d_model=256, num_heads=4, ffn_dim=1024, local_window=64)
    init_block_(blk, std=0.02, seed=3)
    blk = blk.to("cuda", torch.bfloat16)

    def make(i):
        return [_seeded((2, 384, 256), 300 + i)]
    (x,) = make(99)
    with torch.no_grad(), fp8_weight_cache(blk):
        graph, out = _capture(lambda: blk(x))
        _replay_and_compare(graph, out, (x,), make, lambda a: blk(a))


def test_bf16_swa_forward_in_a_graph():
    from flower_amd.kernels.swa_attention import swa_attention
    shape, W = (1, 4, 777, 64), 200

    def make(i):
        return [_seeded(shape, 400 + 10 * i + s) for s in (1, 2, 3)]
    q, k, v = make(99)
    with torch.no_grad():
        graph, out = _capture(lambda: swa_attention(q, k, v, W))
        _replay_and_compare(graph, out, (q, k, v), make, lambda a, b, c: swa_attention(a, b, c, W))


@pytest.mark.parametrize("recipe", [None, "tensorwise"])
def test_training_block_step_in_a_graph(recipe):
    """One training step of the block (flower_amd.block.TransformerBlock: the HIP row kernels, the
    bf16 attention's forward and backward, FP8 or bf16 Linears; forward, then torch.autograd.grad of
    the input and every parameter) captured whole, replayed on new inputs: output and gradients
    equal the eager step's bit for bit."""
    import torch.nn as nn
    from flower_amd.block import TransformerBlock, block_config, init_block_
    from flower_amd.precision import convert_model_to_fp8
    conf = block_config(d_model=256, num_heads=4, ffn_dim=1536, local_window=96, max_seq_len=512)
    blk = init_block_(TransformerBlock(conf), std=0.05, seed=3).to("cuda", torch.bfloat16)
    if recipe is not None:
        stack = nn.Module()
        stack.blocks = nn.ModuleList([blk])
        convert_model_to_fp8(stack, recipe=recipe, keep_bf16_blocks=0, verbose=False)
        blk = stack.blocks[0]
    params = list(blk.parameters())
    shape = (2, 200, 256)

    def make(i):
        return [_seeded(shape, 600 + 10 * i), _seeded(shape, 601 + 10 * i)]

    def step(x, dy):
        xx = x.detach().requires_grad_(True)
        y = blk(xx)[0]
        return [y.detach()] + list(torch.autograd.grad(y, [xx] + params, dy))
    x, dy = make(99)
    graph, out = _capture(lambda: step(x, dy))
    _replay_and_compare(graph, out, (x, dy), make, step)
