"""torch.compile(mode="reduce-overhead"): the compiled block replayed from
graphs (PyTorch's cudagraph trees, HIP graphs on ROCm).

The block's ops are opaque to inductor (their fakes), so their kernels run
inside the captured graph as the ops launch them, workspaces included.  For
the eval forward and for a training step (forward, then backward of
out * up), several inputs of one shape go through the compiled block twice:
the second round (graph replays only) must equal the first bit for bit (whose
first call ran before any graph existed), and every result must agree with
eager mode within the block-level tolerance.  Inductor must not have skipped
the graphs (its cudagraph_skips counter stays at zero).
"""

from __future__ import annotations

import pytest
import torch

import flash_mhc
from parity import block_close

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


def rn(shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV).to(BF16)


def _skips() -> int:
    from torch._dynamo.utils import counters

    return int(counters["inductor"]["cudagraph_skips"])


@pytest.fixture
def replays(monkeypatch):
    """Counts graph replays (cudagraph trees replay through torch.cuda.CUDAGraph.replay)."""
    n = [0]
    orig = torch.cuda.CUDAGraph.replay

    def counted(self):
        n[0] += 1
        return orig(self)

    monkeypatch.setattr(torch.cuda.CUDAGraph, "replay", counted)
    return n


@pytest.mark.parametrize("T", [1, 64, 4096])
def test_reduce_overhead_eval_forward(T, replays):
    C = 1024
    torch.manual_seed(7)
    torch._dynamo.reset()
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).to(DEV, BF16).eval()
    xs = [rn((T, 4, C), 200 + i) for i in range(4)]
    print(f"[reduce-overhead] eval T={T}", flush=True)
    f = torch.compile(blk, mode="reduce-overhead", fullgraph=True)
    skips0 = _skips()
    with torch.no_grad():
        eager = [blk(x) for x in xs]
        rounds = []
        for r in range(2):
            n0 = replays[0]
            outs = []
            for x in xs:
                torch.compiler.cudagraph_mark_step_begin()
                outs.append(f(x).clone())
            rounds.append(outs)
    assert _skips() == skips0, "inductor skipped the graphs"
    assert replays[0] - n0 >= len(xs), "the second round did not replay a graph per call"
    for i in range(len(xs)):
        assert torch.equal(rounds[1][i], rounds[0][i]), f"replay of input {i}"
        block_close(f"reduce-overhead vs eager, input {i}", rounds[1][i], eager[i].float())


@pytest.mark.parametrize("T,ckpt", [(256, False), (4096, False), (4096, True)])
def test_reduce_overhead_training_step(T, ckpt, replays):
    C = 1024
    torch.manual_seed(8)
    torch._dynamo.reset()
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=ckpt)
    blk = blk.to(DEV, BF16)
    data = [(rn((T, 4, C), 300 + i), rn((T, 4, C), 400 + i)) for i in range(3)]
    print(f"[reduce-overhead] training T={T} ckpt={ckpt}", flush=True)

    def step(fn, x, up):
        blk.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        out = fn(xi)
        out.backward(up)
        return [out.detach().clone(), xi.grad.clone()] + [p.grad.clone() for p in blk.parameters()]

    eager = [step(blk, x, up) for x, up in data]
    f = torch.compile(blk, mode="reduce-overhead", fullgraph=True)
    skips0 = _skips()
    rounds = []
    for _ in range(2):
        n0 = replays[0]
        res = []
        for x, up in data:
            torch.compiler.cudagraph_mark_step_begin()
            res.append(step(f, x, up))
        rounds.append(res)
    assert _skips() == skips0, "inductor skipped the graphs"
    # Forward and backward are separate graphs.
    assert replays[0] - n0 >= 2 * len(data), "the second round did not replay the graphs"
    for i in range(len(data)):
        for j, (a, b) in enumerate(zip(rounds[1][i], rounds[0][i])):
            assert torch.equal(a, b), f"replay of step {i}, tensor {j}"
        block_close(f"out {i}", rounds[1][i][0], eager[i][0].float())
        block_close(f"grad_x {i}", rounds[1][i][1], eager[i][1].float(), rtol=5e-2, atol=1e-1)
