"""GPU tests of the fused path at the op and block level.

* autograd through the torch.library ops on the GPU vs the oracle's
  per-op backward values (including K1's grad_W rule);
* the fused bf16 MHCLiteBlock vs the block's fp32 plain formulation (the
  oracle's block_forward): the reference's own end-to-end test shape, the
  golden configuration (T=4096, C=1024, Linear(1024, 1024), loss = sum(out)),
  and the C=2048 configuration with an RMSNorm weight (T=65536);
* torch.compile (inductor, fullgraph) and activation checkpointing;
* eval-mode edge shapes at C=4096, T in {1, 64, 257, 65537}, 1% of tokens x100.

Reference gradients are computed in fp32: torch's batched bf16 products are
avoided on the reference side.
"""

from __future__ import annotations

import copy

import pytest
import torch

import flash_mhc
from oracle import mhc_oracle as O
from parity import block_close, check_bf16, check_fp32

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16 = torch.bfloat16


def randn(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def stress_rows(x, seed, frac=0.01, factor=100.0):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randperm(x.shape[0], generator=g)[: max(1, int(x.shape[0] * frac))]
    y = x.clone()
    y[idx] *= factor
    return y


def fp32_reference(blk: flash_mhc.MHCLiteBlock, device):
    """fp32 leaves + layer copied from `blk`, for the oracle's block formula."""
    p = {
        "W": blk.W_all.weight.detach().float().to(device).clone().requires_grad_(True),
        "b": blk.W_all.bias.detach().float().to(device).clone().requires_grad_(True),
        "alpha_pre": blk.alpha_pre.detach().float().to(device).clone().requires_grad_(True),
        "alpha_post": blk.alpha_post.detach().float().to(device).clone().requires_grad_(True),
        "alpha_res": blk.alpha_res.detach().float().to(device).clone().requires_grad_(True),
        "perm": O.permutation_matrices(4)[0].to(device),
    }
    if blk.rms_weight is not None:
        p["g"] = blk.rms_weight.detach().float().to(device).clone().requires_grad_(True)
    layer = copy.deepcopy(blk.layer).float().to(device)
    return p, layer


def param_grads_ref(p, layer):
    g = {"W_all.weight": p["W"].grad, "W_all.bias": p["b"].grad, "alpha_pre": p["alpha_pre"].grad,
         "alpha_post": p["alpha_post"].grad, "alpha_res": p["alpha_res"].grad}
    if "g" in p:
        g["rms_weight"] = p["g"].grad
    for name, prm in layer.named_parameters():
        g["layer." + name] = prm.grad
    return g


def check_param_grads(blk, pg, taps, tag):
    """Parameter gradients of the fused bf16 block vs the fp32 reference.

    Tensor-valued parameters: relative L2 error < 5e-2.  The scalar alphas:
    each gradient is a sum over all tokens and logits of per-element terms
    that the bf16 pipeline forms from bf16-rounded values (relative error
    ~2^-8 each), and it may be exactly zero in exact arithmetic (sum(out)
    does not depend on alpha_res: the columns of H_res sum to 1, so every
    per-token softmax gradient cancels).  The bar is a 4-sigma random-walk
    bound on those roundings:
        |g - g_ref| <= 5e-2 |g_ref| + 2^-6 * sqrt(sum_terms term^2)
    with terms dL/dz * proj for alpha_pre / alpha_post and, for alpha_res,
    the pre-cancellation softmax terms a * dL/da * proj (fp32 reference)."""
    for name, q in blk.named_parameters():
        ref = pg[name]
        if name.startswith("alpha_"):
            part = name[len("alpha_"):]
            terms = (taps["z_" + part].grad * taps["p_" + part]).abs()
            if part == "res":
                terms = torch.maximum(terms, (taps["a_res"] * taps["a_res"].grad * taps["p_res"]).abs())
            t2 = float(terms.detach().double().pow(2).sum().sqrt())
            err = abs(float(q.grad.float()) - float(ref))
            bound = 5e-2 * abs(float(ref)) + 2.0**-6 * t2
            assert err <= bound, (tag, name, float(q.grad.float()), float(ref), t2)
        else:
            assert rel_l2(q.grad, ref) < 5e-2, (tag, name, rel_l2(q.grad, ref))


def rel_l2(a, b) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


class GeluLinear(torch.nn.Module):
    """The reference's E2E inner layer (tests/test_correctness.py:320-329)."""

    def __init__(self, dim):
        super().__init__()
        self.proj = torch.nn.Linear(dim, dim, bias=False)

    def forward(self, x, **kwargs):
        return torch.nn.functional.gelu(self.proj(x))


# ---------------------------------------------------------------------------
# ops + autograd


def test_op_autograd_matches_oracle():
    T, C = 1024, 256
    nC = 4 * C
    x = randn((T, 4, C), 1, dtype=BF16)
    W = randn((32, nC), 2, 0.02, dtype=BF16)
    h = torch.sigmoid(randn((T, 4), 3))
    lo = randn((T, C), 4, dtype=BF16)
    H = randn((T, 4, 4), 5)
    hp = randn((T, 4), 6)
    go1, go3, go4 = randn((T, 32), 7, dtype=BF16), randn((T, C), 8, dtype=BF16), randn((T, 4, C), 9, dtype=BF16)

    xs = x.to(DEV).reshape(T, nC).requires_grad_(True)
    Ws = W.to(DEV).requires_grad_(True)
    proj, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xs, Ws)
    proj.backward(go1.to(DEV))
    R, S = O.k1_bwd_dx(go1, x.view(T, nC), W, proj.detach().cpu(), inv.cpu())
    check_bf16("op k1 grad_x", xs.grad, R, S, 64)
    R, S = O.k1_grad_W(go1, x.view(T, nC), inv.cpu())
    check_bf16("op k1 grad_W", Ws.grad, R, S, T)

    xs = x.to(DEV).requires_grad_(True)
    hs = h.to(DEV).requires_grad_(True)
    torch.ops.flash_mhc.fused_pre_map(xs, hs).backward(go3.to(DEV))
    gxR, gxS, ghR, ghS = O.k3_bwd(go3, x, h)
    check_bf16("op k3 grad_x", xs.grad, gxR, gxS, 1)
    check_fp32("op k3 grad_h", hs.grad, ghR, ghS, C)

    leaves = [t.to(DEV).requires_grad_(True) for t in (x, lo, H, hp)]
    torch.ops.flash_mhc.fused_post_res(*leaves).backward(go4.to(DEV))
    ref = O.k4_bwd(go4, x, lo, H, hp)
    check_bf16("op k4 grad_x", leaves[0].grad, *ref["grad_x"], 4)
    check_bf16("op k4 grad_lo", leaves[1].grad, *ref["grad_lo"], 4)
    check_fp32("op k4 grad_H", leaves[2].grad, *ref["grad_H"], C)
    check_fp32("op k4 grad_hp", leaves[3].grad, *ref["grad_hp"], C)


def test_ops_reject_bad_inputs_on_gpu():
    x = torch.zeros(8, 3, 16, dtype=BF16, device=DEV)
    with pytest.raises(ValueError, match="n=4 only"):
        torch.ops.flash_mhc.fused_pre_map(x, torch.zeros(8, 3, device=DEV))
    with pytest.raises(TypeError):
        torch.ops.flash_mhc.fused_pre_map(torch.zeros(8, 4, 16, device=DEV), torch.zeros(8, 4, device=DEV))
    with pytest.raises(ValueError):
        torch.ops.flash_mhc.fused_rmsnorm_project(torch.zeros(8, 64, dtype=BF16, device=DEV),
                                                  torch.zeros(31, 64, dtype=BF16, device=DEV))


# ---------------------------------------------------------------------------
# block vs fp32 reference


def _run_pair(blk_bf16, x_cpu, device_ref, upstream=None, ref_on=DEV):
    """Fused bf16 forward+backward and the fp32 reference on the same input."""
    x = x_cpu.to(DEV, BF16).requires_grad_(True)
    out = blk_bf16(x)
    gout = torch.ones_like(out) if upstream is None else upstream.to(DEV, BF16)
    out.backward(gout)
    p, layer = device_ref
    xr = x_cpu.to(BF16).float().to(ref_on).requires_grad_(True)  # same rounded input
    taps = {}
    ref = O.block_forward(xr, p, layer, 4, taps)
    ref.backward(torch.ones_like(ref) if upstream is None else upstream.to(BF16).float().to(ref_on))
    return out, x.grad, ref, xr.grad, param_grads_ref(p, layer), taps


def test_block_reference_e2e_shape():
    """Shape and layer of the reference's TestMHCLiteBlockEndToEnd (T=1024, C=256)."""
    torch.manual_seed(0)
    C = 256
    blk = flash_mhc.MHCLiteBlock(4, C, GeluLinear(C)).to(DEV, BF16)
    ref = fp32_reference(blk, DEV)
    x = randn((1024, 4, C), 11)
    out, gx, r, gr, pg, taps = _run_pair(blk, x, ref)
    block_close("e2e out", out, r)
    block_close("e2e grad_x", gx, gr, rtol=5e-2, atol=1e-1)
    check_param_grads(blk, pg, taps, "e2e")


def test_block_golden_config():
    """T=4096, n=4, C=1024, bias-free Linear(1024,1024), x ~ N(0,1) seed 0,
    loss sum(out); reference: fp32 plain formulation on the CPU."""
    torch.manual_seed(0)
    C = 1024
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).to(DEV, BF16)
    ref = fp32_reference(blk, "cpu")
    x = torch.randn(4096, 4, C, generator=torch.Generator().manual_seed(0))
    out, gx, r, gr, pg, taps = _run_pair(blk, x, ref, ref_on="cpu")
    block_close("golden out", out, r)
    block_close("golden grad_x", gx, gr, rtol=5e-2, atol=1e-1)
    check_param_grads(blk, pg, taps, "golden")


def test_block_c2048_rmsnorm_weight():
    """T=65536, n=4, C=2048, Linear(2048, 2048), upstream grad ~ N(0,1); dx,
    dW_proj and d(RMSNorm weight) against fp32."""
    torch.manual_seed(0)
    C, T = 2048, 65536
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), rmsnorm_weight=True)
    with torch.no_grad():
        blk.rms_weight.copy_(1 + 0.02 * torch.randn(4 * C))
    blk = blk.to(DEV, BF16)
    ref = fp32_reference(blk, DEV)
    x = randn((T, 4, C), 21)
    up = randn((T, 4, C), 22)
    out, gx, r, gr, pg, taps = _run_pair(blk, x, ref, upstream=up)
    block_close("c2048 out", out, r)
    block_close("c2048 grad_x", gx, gr, rtol=5e-2, atol=1e-1)
    assert rel_l2(blk.W_all.weight.grad, pg["W_all.weight"]) < 5e-2
    assert rel_l2(blk.rms_weight.grad, pg["rms_weight"]) < 5e-2
    check_param_grads(blk, pg, taps, "c2048")


@pytest.mark.parametrize("T", [1, 64, 257, 65537])
def test_eval_edge_shapes(T):
    torch.manual_seed(0)
    C = 4096
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).to(DEV, BF16).eval()
    p, layer = fp32_reference(blk, DEV)
    x = stress_rows(randn((T, 4, C), 30 + T), 31 + T)
    with torch.no_grad():
        out = blk(x.to(DEV, BF16))
        ref = O.block_forward(x.to(BF16).float().to(DEV), p, layer, 4)
    block_close(f"eval T={T}", out, ref)


# ---------------------------------------------------------------------------
# torch.compile and activation checkpointing


def test_torch_compile_inductor():
    torch.manual_seed(0)
    C = 256
    blk = flash_mhc.MHCLiteBlock(4, C, GeluLinear(C)).to(DEV, BF16)
    ref = fp32_reference(blk, DEV)
    x = randn((1024, 4, C), 41)

    xe = x.to(DEV, BF16).requires_grad_(True)
    oe = blk(xe)
    oe.float().sum().backward()
    ge = {n: q.grad.clone() for n, q in blk.named_parameters()}
    blk.zero_grad()

    compiled = torch.compile(blk, fullgraph=True)
    xc = x.to(DEV, BF16).requires_grad_(True)
    oc = compiled(xc)
    oc.float().sum().backward()
    p, layer = ref
    xr = x.to(BF16).float().to(DEV).requires_grad_(True)
    taps = {}
    rr = O.block_forward(xr, p, layer, 4, taps)
    rr.sum().backward()
    block_close("compiled out vs fp32", oc, rr)
    block_close("compiled grad_x vs fp32", xc.grad, xr.grad, rtol=5e-2, atol=1e-1)
    block_close("compiled vs eager out", oc, oe)
    block_close("compiled vs eager grad_x", xc.grad, xe.grad, rtol=5e-2, atol=1e-1)
    check_param_grads(blk, param_grads_ref(p, layer), taps, "compiled")


def test_activation_checkpointing_same_grads():
    torch.manual_seed(0)
    C = 512
    blk = flash_mhc.MHCLiteBlock(4, C, GeluLinear(C)).to(DEV, BF16)
    x = randn((2048, 4, C), 51).to(DEV, BF16)
    up = randn((2048, 4, C), 52).to(DEV, BF16)
    res = []
    for ckpt in (False, True):
        blk.activation_checkpointing = ckpt
        blk.zero_grad()
        xi = x.clone().requires_grad_(True)
        out = blk(xi)
        out.backward(up)
        res.append((out.detach(), xi.grad, {n: q.grad.clone() for n, q in blk.named_parameters()}))
    (o0, g0, p0), (o1, g1, p1) = res
    assert torch.equal(o0, o1)
    assert torch.equal(g0, g1)
    for n in p0:
        assert torch.equal(p0[n], p1[n]), n


@pytest.mark.parametrize("T", [1, 64, 4096])
def test_graph_capture_eval_forward(T):
    """The fused block's eval forward (K1, K2, K3 on the pre-map op, the layer,
    K4) can be captured in a HIP graph: every replay, with eager work and
    synchronisations between replays, equals the eager forward."""
    C = 1024
    torch.manual_seed(3)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False)).to(DEV, BF16).eval()
    x = randn((T, 4, C), 70 + T, dtype=BF16).to(DEV)
    with torch.no_grad():
        ref = blk(x).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                blk(x)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = blk(x)
        for i in range(4):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {i}"
            eager = blk(x)  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(eager, ref)


@pytest.mark.parametrize("T,rms", [(256, False), (4096, True), (20000, False)])
def test_eager_autograd_path_equals_op_path(T, rms):
    """In eager training the block applies mhc_pre_map and mhc_post_res as
    autograd Functions around the ops' device implementations.  Its output,
    x's gradient and every parameter gradient equal, bit for bit, those of
    the same block driven through the torch.library ops (T = 20000: the
    one-kernel pre-map forward)."""
    from contextlib import nullcontext

    C = 1024
    torch.manual_seed(5)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), rmsnorm_weight=rms).to(DEV, BF16)
    if rms:
        with torch.no_grad():
            blk.rms_weight.add_(randn((4 * C,), 96, 0.02).to(DEV, blk.rms_weight.dtype))
    x = randn((T, 4, C), 97 + T, dtype=BF16).to(DEV)
    up = randn((T, 4, C), 98 + T, dtype=BF16).to(DEV)

    def run(fast):
        blk.zero_grad(set_to_none=True)
        xs = x.clone().requires_grad_(True)
        if fast:
            out = blk(xs)
        else:
            out = blk._run(xs, blk._mhc_pre_map_triton, blk._mhc_post_res_triton, nullcontext(), {},
                           checkpoint_post_res=False)
        out.backward(up)
        return [out.detach(), xs.grad] + [p.grad.clone() for p in blk.parameters()]

    fast, ops = run(True), run(False)
    names = ["out", "grad_x"] + [n for n, _ in blk.named_parameters()]
    for name, a, b in zip(names, fast, ops):
        assert torch.equal(a, b), f"{name} differs"


@pytest.mark.parametrize("T,ckpt", [(256, False), (4096, False), (256, True)])
def test_graph_capture_training_step(T, ckpt):
    """A whole training step of the fused block (forward, then backward of
    out * up) captured in one HIP graph: for new inputs copied into the
    captured buffers, every replay gives the eager step's output and
    gradients bit for bit, with eager steps between the replays."""
    C = 1024
    torch.manual_seed(4)
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=ckpt).to(DEV, BF16)
    sx = randn((T, 4, C), 80 + T, dtype=BF16).to(DEV).requires_grad_(True)
    sup = randn((T, 4, C), 81 + T, dtype=BF16).to(DEV)

    def step(x, up):
        blk.zero_grad(set_to_none=True)
        x.grad = None
        out = blk(x)
        out.backward(up)
        return out

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            step(sx, sup)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    blk.zero_grad(set_to_none=True)
    sx.grad = None
    # Captured on the warm-up's stream: the parameters' AccumulateGrad nodes
    # keep the stream of their first backward, and a capture on another one
    # makes autograd add cross-stream syncs (and warn).
    with torch.cuda.graph(g, stream=s):
        sout = blk(sx)
        sout.backward(sup)
    # Keep only the output buffer: a live reference to the captured autograd
    # graph would keep its AccumulateGrad nodes (stream s) for the eager
    # steps below, which run on the default stream.
    sout = sout.detach()
    # The gradients the captured backward writes (the eager steps below
    # attach new ones to the parameters).
    names = [n for n, _ in blk.named_parameters()]
    sgrads = [sx.grad] + [p.grad for p in blk.parameters()]
    for i in range(3):
        x = randn((T, 4, C), 90 + 7 * i + T, dtype=BF16).to(DEV)
        up = randn((T, 4, C), 91 + 7 * i + T, dtype=BF16).to(DEV)
        with torch.no_grad():
            sx.copy_(x)
            sup.copy_(up)
        g.replay()
        torch.cuda.synchronize()
        got = [sout.detach().clone()] + [t.clone() for t in sgrads]
        xe = x.clone().requires_grad_(True)
        oute = step(xe, up)  # eager step between replays, on other buffers
        torch.cuda.synchronize()
        want = [oute.detach(), xe.grad] + [p.grad for p in blk.parameters()]
        for name, a, b in zip(["out", "grad_x"] + names, got, want):
            assert torch.equal(a, b), f"replay {i}: {name} differs"


@pytest.mark.parametrize("ckpt", [False, True])
def test_empty_batch_forward_backward(ckpt):
    """T = 0 through the fused block, training and eval: empty outputs, an empty
    x gradient and zero parameter gradients."""
    torch.manual_seed(0)
    C = 256
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), activation_checkpointing=ckpt).to(DEV, BF16)
    x = torch.empty((0, 4, C), device=DEV, dtype=BF16, requires_grad=True)
    out = blk(x)
    assert out.shape == (0, 4, C)
    out.float().sum().backward()
    assert x.grad.shape == (0, 4, C)
    for name, p in blk.named_parameters():
        assert p.grad is None or float(p.grad.float().abs().sum()) == 0.0, name
    with torch.no_grad():
        assert blk.eval()(x.detach()).shape == (0, 4, C)


def _mixed_block(C, fp32_params: bool, rms: bool):
    """A fused-path block: bf16 throughout, or with its own parameters (W_all,
    alphas, the RMSNorm weight) in fp32 and only the layer in bf16."""
    blk = flash_mhc.MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), rmsnorm_weight=rms).to(DEV)
    if rms:
        with torch.no_grad():
            blk.rms_weight.add_(randn((4 * C,), 71, 0.02).to(DEV))
    if fp32_params:
        blk.layer.to(BF16)
    else:
        blk.to(BF16)
    return blk


@pytest.mark.parametrize("T,C,fp32_params,rms", [(1, 4096, False, False), (64, 4096, False, False),
                                                  (257, 1024, False, False), (5000, 1024, False, False),
                                                  (333, 100, False, False), (64, 4096, True, False),
                                                  (20000, 1024, True, True), (257, 1024, False, True)])
def test_nograd_forward_equals_op_path(T, C, fp32_params, rms):
    """Without autograd the block launches the pre-map and post-res kernels
    directly (no custom-op dispatch): the same bits as the block driven through
    the torch.library ops, in eval and in training mode, with bf16 or fp32
    block parameters and with the RMSNorm weight."""
    from contextlib import nullcontext

    torch.manual_seed(7)
    blk = _mixed_block(C, fp32_params, rms)
    x = randn((T, 4, C), 70 + T, dtype=BF16).to(DEV)
    for training in (False, True):
        blk.train(training)
        with torch.no_grad():
            fast = blk(x)
            ops_path = blk._run(x, blk._mhc_pre_map_triton, blk._mhc_post_res_triton, nullcontext(), {},
                                checkpoint_post_res=False)
        torch.cuda.synchronize()
        assert torch.equal(fast, ops_path), (T, C, training)


@pytest.mark.parametrize("T,C", [(64, 4096), (5000, 1024)])
def test_eager_autograd_path_fp32_params_equals_op_path(T, C):
    """The eager autograd path with fp32 block parameters (bf16 layer) and
    the RMSNorm weight: output and every gradient equal the op path's."""
    from contextlib import nullcontext

    torch.manual_seed(8)
    blk = _mixed_block(C, True, True)
    x = randn((T, 4, C), 72 + T, dtype=BF16).to(DEV)
    up = randn((T, 4, C), 73 + T, dtype=BF16).to(DEV)

    def run(fast):
        blk.zero_grad(set_to_none=True)
        xs = x.clone().requires_grad_(True)
        out = blk(xs) if fast else blk._run(xs, blk._mhc_pre_map_triton, blk._mhc_post_res_triton,
                                            nullcontext(), {}, checkpoint_post_res=False)
        out.backward(up)
        return [out.detach(), xs.grad] + [p.grad.clone() for p in blk.parameters()]

    names = ["out", "grad_x"] + [n for n, _ in blk.named_parameters()]
    for name, a, b in zip(names, run(True), run(False)):
        assert a.dtype == b.dtype and torch.equal(a, b), f"{name} differs"
