"""CPU tests of the flash_mhc op boundary (torch.library contract).

The schema strings, fake-tensor shapes and autograd behaviour must be the
reference's (src/flash_mhc/ops.py:22-41, :145-202, :670-714).  Device work is
replaced here by the oracle's CPU kernels (tests/oracle_cpu_ops.py) so the
contract is exercised without a GPU; GPU parity is in test_gpu_*.py.
"""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import flash_mhc
from flash_mhc import kernels as K
from flash_mhc import ops
from oracle import mhc_oracle as O
from oracle_cpu_ops import oracle_cpu_kernels

BF16 = torch.bfloat16

# Verbatim from the reference (ops.py:24-41).
REFERENCE_SCHEMAS = {
    "fused_rmsnorm_project": "fused_rmsnorm_project(Tensor x_flat, Tensor W) -> (Tensor out, Tensor inv_rms)",
    "fused_rmsnorm_project_bwd_dx": "fused_rmsnorm_project_bwd_dx(Tensor grad_out, Tensor x_flat, Tensor W, Tensor proj_out, Tensor inv_rms) -> Tensor grad_x",
    "fused_pre_map": "fused_pre_map(Tensor x_streams, Tensor h_pre) -> Tensor out",
    "fused_pre_map_backward": "fused_pre_map_backward(Tensor grad_out, Tensor x_streams, Tensor h_pre) -> (Tensor grad_x, Tensor grad_h_pre)",
    "fused_post_res": "fused_post_res(Tensor x_streams, Tensor layer_output, Tensor H_merged, Tensor h_post) -> Tensor out",
    "fused_post_res_backward": "fused_post_res_backward(Tensor grad_out, Tensor x_streams, Tensor layer_output, Tensor H_merged, Tensor h_post) -> (Tensor grad_x, Tensor grad_layer_output, Tensor grad_H_merged, Tensor grad_h_post)",
}


def rnd(shape, seed, scale=1.0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schema_matches_reference(name):
    op = getattr(torch.ops.flash_mhc, name).default
    assert str(op._schema) == "flash_mhc::" + REFERENCE_SCHEMAS[name]


def test_fused_backward_op_contract():
    op = torch.ops.flash_mhc.fused_rmsnorm_project_bwd.default
    assert str(op._schema) == ("flash_mhc::fused_rmsnorm_project_bwd(Tensor grad_out, Tensor x_flat, "
                               "Tensor W, Tensor proj_out, Tensor inv_rms) -> (Tensor grad_x, Tensor grad_W)")
    assert torch._C._dispatch_has_kernel_for_dispatch_key("flash_mhc::fused_rmsnorm_project_bwd", "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key("flash_mhc::fused_rmsnorm_project_bwd", "CPU")
    with FakeTensorMode():
        xf = torch.empty(7, 96, dtype=BF16)
        W = torch.empty(32, 96, dtype=BF16)
        g = torch.empty(7, 32, dtype=BF16)
        gx, gW = torch.ops.flash_mhc.fused_rmsnorm_project_bwd(g, xf, W, g, torch.empty(7))
        assert gx.shape == xf.shape and gx.dtype == BF16 and gW.shape == W.shape and gW.dtype == BF16


ADDED_SCHEMAS = {
    "fused_rmsnorm_project_bwd": "fused_rmsnorm_project_bwd(Tensor grad_out, Tensor x_flat, Tensor W, Tensor proj_out, Tensor inv_rms) -> (Tensor grad_x, Tensor grad_W)",
    "mhc_coefficients": "mhc_coefficients(Tensor proj, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor h_pre, Tensor h_post, Tensor H_merged)",
    "mhc_coefficients_backward": "mhc_coefficients_backward(Tensor? grad_h_pre, Tensor? grad_h_post, Tensor? grad_H_merged, Tensor proj, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor grad_proj, Tensor grad_alpha_pre, Tensor grad_alpha_post, Tensor grad_alpha_res, Tensor grad_bias)",
    "mhc_pre_map": "mhc_pre_map(Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor layer_input, Tensor H_merged, Tensor h_post, Tensor h_pre, Tensor proj, Tensor inv_rms, Tensor x_sink)",
    "mhc_pre_map_backward": "mhc_pre_map_backward(Tensor? grad_layer_input, Tensor? grad_H_merged, Tensor? grad_h_post, Tensor? grad_h_pre, Tensor? grad_proj, Tensor? grad_x_sink, Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat, Tensor h_pre, Tensor proj, Tensor inv_rms) -> (Tensor grad_x, Tensor grad_W, Tensor grad_alpha_pre, Tensor grad_alpha_post, Tensor grad_alpha_res, Tensor grad_bias)",
    "mhc_post_res": "mhc_post_res(Tensor x_streams, Tensor x_sink, Tensor layer_output, Tensor H_merged, Tensor h_post) -> Tensor out",
    "mhc_pre_map_coeffs": "mhc_pre_map_coeffs(Tensor x_streams, Tensor W, Tensor alpha_pre, Tensor alpha_post, Tensor alpha_res, Tensor bias, Tensor perm_mat) -> (Tensor H_merged, Tensor h_post, Tensor h_pre, Tensor proj, Tensor inv_rms, Tensor x_sink, Tensor li_sink)",
    "mhc_pre_map_mix": "mhc_pre_map_mix(Tensor x_streams, Tensor h_pre, Tensor li_sink) -> Tensor layer_input",
}


@pytest.mark.parametrize("name", sorted(ADDED_SCHEMAS))
def test_added_ops_device_only(name):
    op = getattr(torch.ops.flash_mhc, name).default
    assert str(op._schema) == "flash_mhc::" + ADDED_SCHEMAS[name]
    assert torch._C._dispatch_has_kernel_for_dispatch_key(f"flash_mhc::{name}", "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(f"flash_mhc::{name}", "CPU")


def test_mhc_coefficients_fakes_and_n4_error():
    with FakeTensorMode():
        proj = torch.empty(7, 32, dtype=BF16)
        a = torch.empty(1)
        hp, hq, H = torch.ops.flash_mhc.mhc_coefficients(proj, a, a, a, torch.empty(32), torch.empty(24, 16))
        assert hp.shape == (7, 4) and hq.shape == (7, 4) and H.shape == (7, 4, 4)
        assert hp.dtype == hq.dtype == H.dtype == torch.float32
        g = torch.ops.flash_mhc.mhc_coefficients_backward(hp, None, H, proj, a, a, a, torch.empty(32),
                                                          torch.empty(24, 16))
        assert g[0].shape == proj.shape and g[0].dtype == BF16 and g[4].shape == (32,)
    with pytest.raises(ValueError, match="n=4 only"):
        ops._mhc_coefficients_cuda(torch.empty(3, 12, dtype=BF16), *[torch.empty(1)] * 3, torch.empty(12),
                                   torch.empty(6, 9))


def test_only_device_kernels_registered():
    """No CPU implementation ships: the device path cannot silently fall back."""
    for name in REFERENCE_SCHEMAS:
        qual = f"flash_mhc::{name}"
        assert torch._C._dispatch_has_kernel_for_dispatch_key(qual, "CUDA")
        assert not torch._C._dispatch_has_kernel_for_dispatch_key(qual, "CPU")
    with pytest.raises(NotImplementedError):
        torch.ops.flash_mhc.fused_pre_map(rnd((2, 4, 8), 0), torch.zeros(2, 4))


def test_fakes():
    with FakeTensorMode():
        T, C = 7, 24
        x = torch.empty(T, 4, C, dtype=BF16)
        xf = torch.empty(T, 4 * C, dtype=BF16)
        W = torch.empty(32, 4 * C, dtype=BF16)
        out, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xf, W)
        assert out.shape == (T, 32) and out.dtype == BF16 and inv.shape == (T,) and inv.dtype == torch.float32
        gx = torch.ops.flash_mhc.fused_rmsnorm_project_bwd_dx(out, xf, W, out, inv)
        assert gx.shape == xf.shape and gx.dtype == BF16
        h = torch.empty(T, 4, dtype=BF16)
        li = torch.ops.flash_mhc.fused_pre_map(x, h)
        assert li.shape == (T, C) and li.dtype == BF16
        gx, gh = torch.ops.flash_mhc.fused_pre_map_backward(li, x, h)
        assert gx.shape == x.shape and gh.shape == (T, 4) and gh.dtype == torch.float32
        lo = torch.empty(T, C, dtype=BF16)
        H = torch.empty(T, 4, 4)
        hp = torch.empty(T, 4)
        o = torch.ops.flash_mhc.fused_post_res(x, lo, H, hp)
        assert o.shape == x.shape and o.dtype == BF16
        g = torch.ops.flash_mhc.fused_post_res_backward(o, x, lo, H, hp)
        assert [t.shape for t in g] == [x.shape, lo.shape, H.shape, hp.shape]
        assert [t.dtype for t in g] == [BF16, BF16, torch.float32, torch.float32]


@pytest.mark.parametrize(
    "fn,args,msg",
    [
        (ops._fused_pre_map_cuda, lambda: (rnd((2, 3, 8), 1), torch.zeros(2, 3)),
         "flash_mhc::fused_pre_map currently supports n=4 only"),
        (ops._fused_pre_map_backward_cuda, lambda: (rnd((2, 8), 1), rnd((2, 3, 8), 1), torch.zeros(2, 3)),
         "flash_mhc::fused_pre_map_backward supports n=4 only"),
        (ops._fused_post_res_cuda, lambda: (rnd((2, 5, 8), 1), rnd((2, 8), 1), torch.zeros(2, 5, 5), torch.zeros(2, 5)),
         "flash_mhc::fused_post_res currently supports n=4 only"),
        (ops._fused_post_res_backward_cuda,
         lambda: (rnd((2, 5, 8), 1), rnd((2, 5, 8), 1), rnd((2, 8), 1), torch.zeros(2, 5, 5), torch.zeros(2, 5)),
         "flash_mhc::fused_post_res_backward supports n=4 only"),
    ],
)
def test_n_not_4_errors_match_reference(fn, args, msg):
    with pytest.raises(ValueError, match=msg):
        fn(*args())


def test_launchers_reject_host_tensors_and_bad_args():
    x = rnd((4, 4, 8), 2)
    with pytest.raises(ValueError, match="GPU tensor"):
        K.k3_fwd(x, torch.zeros(4, 4))
    with pytest.raises(ValueError, match="GPU tensor"):
        K.k1_fwd(x.view(4, 32), rnd((32, 32), 3))
    with pytest.raises(TypeError):
        K.k3_fwd("not a tensor", None)


def test_disable_autotune_context_is_a_reentrant_no_op():
    """The reference's context manager (ops.py:44-58) exists for callers that
    enter it; with fixed launch configurations it nests and does nothing."""
    with ops.disable_autotune_temporarily():
        with ops.disable_autotune_temporarily():
            pass
    with pytest.raises(KeyError):  # exceptions pass through unchanged
        with ops.disable_autotune_temporarily():
            raise KeyError("x")


# ---------------------------------------------------------------------------
# With the oracle standing in for the device kernels


@pytest.fixture
def cpu_kernels():
    with oracle_cpu_kernels():
        yield


def _samples():
    T, C = 6, 16
    x = rnd((T, 4, C), 10)
    xf = x.reshape(T, 4 * C)
    W = rnd((32, 4 * C), 11, 0.05)
    h = torch.rand(T, 4, generator=torch.Generator().manual_seed(12))
    lo = rnd((T, C), 13)
    H = rnd((T, 4, 4), 14, dtype=torch.float32)
    hp = rnd((T, 4), 15, dtype=torch.float32)
    return T, C, x, xf, W, h, lo, H, hp


def test_opcheck_all_ops(cpu_kernels):
    T, C, x, xf, W, h, lo, H, hp = _samples()
    proj, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xf, W)
    cases = [
        (torch.ops.flash_mhc.fused_rmsnorm_project.default, (xf.clone().requires_grad_(True), W.clone().requires_grad_(True))),
        (torch.ops.flash_mhc.fused_rmsnorm_project_bwd_dx.default, (rnd((T, 32), 16), xf, W, proj, inv)),
        (torch.ops.flash_mhc.fused_rmsnorm_project_bwd.default, (rnd((T, 32), 16), xf, W, proj, inv)),
        (torch.ops.flash_mhc.fused_pre_map.default, (x.clone().requires_grad_(True), h.clone().requires_grad_(True))),
        (torch.ops.flash_mhc.fused_pre_map_backward.default, (rnd((T, C), 17), x, h)),
        (torch.ops.flash_mhc.fused_post_res.default,
         (x.clone().requires_grad_(True), lo.clone().requires_grad_(True), H.clone().requires_grad_(True), hp.clone().requires_grad_(True))),
        (torch.ops.flash_mhc.fused_post_res_backward.default, (rnd((T, 4, C), 18), x, lo, H, hp)),
    ]
    k2p = [torch.tensor([0.7]), torch.tensor([1.1]), torch.tensor([1.9]), rnd((32,), 19, 0.5, torch.float32)]
    perm = O.permutation_matrices(4)[0]
    cases += [
        (torch.ops.flash_mhc.mhc_coefficients.default,
         (proj.clone().requires_grad_(True), *[t.clone().requires_grad_(True) for t in k2p], perm)),
        (torch.ops.flash_mhc.mhc_coefficients_backward.default,
         (hp, None, H, proj, *k2p, perm)),
        (torch.ops.flash_mhc.mhc_pre_map.default,
         (x.clone().requires_grad_(True), W.clone().requires_grad_(True),
          *[t.clone().requires_grad_(True) for t in k2p], perm)),
    ]
    li, H2, hq2, hp2, proj2, inv2, sink = torch.ops.flash_mhc.mhc_pre_map(x, W, *k2p, perm)
    assert sink.shape == x.shape and sink.stride() == (0, 0, 0) and sink.dtype == x.dtype
    cases += [
        (torch.ops.flash_mhc.mhc_pre_map_backward.default,
         (rnd((T, C), 22), H, hp, None, None, None, x, W, *k2p, perm, hp2, proj2, inv2)),
        (torch.ops.flash_mhc.mhc_pre_map_backward.default,
         (rnd((T, C), 22), H, hp, None, None, rnd((T, 4, C), 23), x, W, *k2p, perm, hp2, proj2, inv2)),
        (torch.ops.flash_mhc.mhc_post_res.default,
         (x.clone().requires_grad_(True), sink.clone().requires_grad_(True), lo.clone().requires_grad_(True),
          H.clone().requires_grad_(True), hp.clone().requires_grad_(True))),
        (torch.ops.flash_mhc.mhc_pre_map_coeffs.default,
         (x.clone().requires_grad_(True), W.clone().requires_grad_(True),
          *[t.clone().requires_grad_(True) for t in k2p], perm)),
    ]
    outs = torch.ops.flash_mhc.mhc_pre_map_coeffs(x, W, *k2p, perm)
    assert outs[6].shape == (T, C) and outs[6].stride() == (0, 0)
    cases.append((torch.ops.flash_mhc.mhc_pre_map_mix.default,
                  (x.clone().requires_grad_(True), outs[2].clone().requires_grad_(True),
                   outs[6].clone().requires_grad_(True))))
    for op, args in cases:
        torch.library.opcheck(op, args)


@pytest.mark.parametrize("fused", ["1", "0"])
def test_k1_autograd_rules_agree(cpu_kernels, monkeypatch, fused):
    """The fused K1 backward op and the reference's two-step rule give the
    same gradients (bf16 rounding of grad_W aside)."""
    monkeypatch.setenv("FLASH_MHC_FUSED_DW", fused)
    T, C, x, xf, W, h, lo, H, hp = _samples()
    xs = xf.clone().requires_grad_(True)
    Ws = W.clone().requires_grad_(True)
    proj, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xs, Ws)
    go1 = rnd((T, 32), 21)
    proj.backward(go1)
    gx, _ = O.k1_bwd_dx(go1, xf, W, proj.detach(), inv)
    gW, _ = O.k1_grad_W(go1, xf, inv)
    assert torch.equal(xs.grad, gx.to(BF16))
    torch.testing.assert_close(Ws.grad.double(), gW, rtol=1e-2, atol=1e-2)


def test_autograd_formulas(cpu_kernels):
    """Gradients through the ops equal the oracle's backward values."""
    T, C, x, xf, W, h, lo, H, hp = _samples()
    xs = x.clone().requires_grad_(True)
    hs = h.clone().requires_grad_(True)
    go3 = rnd((T, C), 20)
    torch.ops.flash_mhc.fused_pre_map(xs, hs).backward(go3)
    gx, _, gh, _ = O.k3_bwd(go3, x, h)
    assert torch.equal(xs.grad, gx.to(BF16))
    torch.testing.assert_close(hs.grad, gh.float())

    xs = xf.clone().requires_grad_(True)
    Ws = W.clone().requires_grad_(True)
    proj, inv = torch.ops.flash_mhc.fused_rmsnorm_project(xs, Ws)
    go1 = rnd((T, 32), 21)
    proj.backward(go1)
    gx, _ = O.k1_bwd_dx(go1, xf, W, proj.detach(), inv)
    gW, _ = O.k1_grad_W(go1, xf, inv)
    assert torch.equal(xs.grad, gx.to(BF16))
    torch.testing.assert_close(Ws.grad.double(), gW, rtol=1e-2, atol=1e-2)


def _block(seed=0, C=16):
    torch.manual_seed(seed)
    layer = torch.nn.Sequential(torch.nn.Linear(C, C, bias=False), torch.nn.GELU())
    return flash_mhc.MHCLiteBlock(4, C, layer).to(BF16)


def test_compile_fullgraph_fused_block(cpu_kernels):
    """The fused block traces under torch.compile(fullgraph=True) with no graph
    breaks, and compiled forward + backward equal eager."""
    blk = _block()
    x = rnd((8, 4, 16), 30)
    xe = x.clone().requires_grad_(True)
    out_e = blk._forward_triton(xe)
    out_e.float().sum().backward()
    ge = {n: p.grad.clone() for n, p in blk.named_parameters()}
    blk.zero_grad()
    compiled = torch.compile(blk._forward_triton, fullgraph=True, backend="aot_eager")
    xc = x.clone().requires_grad_(True)
    out_c = compiled(xc)
    out_c.float().sum().backward()
    assert torch.equal(out_c, out_e)
    assert torch.equal(xc.grad, xe.grad)
    for n, p in blk.named_parameters():
        assert torch.equal(p.grad, ge[n]), n


def test_fused_block_matches_plain_block_on_cpu(cpu_kernels):
    """The fused composition (K1 project-then-normalise, K2 in bf16, K3, K4)
    agrees with the block's plain formulation to bf16 accuracy."""
    from parity import block_close

    blk = _block(C=32)
    x = rnd((64, 4, 32), 31)
    with torch.no_grad():
        a = blk._forward_triton(x)
        b = blk.float()._forward_pytorch(x.float())
    block_close("fused vs plain", a, b)


def test_fused_k2_matches_reference_chain_on_cpu(cpu_kernels, monkeypatch):
    """The block with K2 as one op (FLASH_MHC_FUSED_K2=1) and with the
    reference's PyTorch ops (=0) give the same outputs and gradients: the op's
    autograd wiring routes every gradient to the right parameter."""

    def run(flag):
        monkeypatch.setenv("FLASH_MHC_FUSED_K2", flag)
        monkeypatch.setenv("FLASH_MHC_FUSED_PREMAP", "0")
        blk = _block(C=32)
        with torch.no_grad():
            blk.alpha_pre.fill_(0.8)
            blk.alpha_post.fill_(1.2)
            blk.alpha_res.fill_(1.7)
        x = rnd((64, 4, 32), 41).requires_grad_(True)
        out = blk._forward_triton(x)
        out.float().pow(2).sum().backward()
        return out.detach(), x.grad, {n: p.grad for n, p in blk.named_parameters()}

    from parity import block_close

    o1, gx1, gp1 = run("1")
    o0, gx0, gp0 = run("0")
    assert torch.equal(o1, o0)
    # The op rounds the sigmoid / softmax backward steps as torch's GPU kernels
    # do, the CPU chain as torch's CPU kernels do: gradients agree to bf16
    # accuracy (the reference's end-to-end gradient tolerance, per token).
    block_close("grad_x fused K2 vs ops", gx1.float(), gx0.float(), rtol=5e-2, atol=1e-1)
    for n in gp0:
        torch.testing.assert_close(gp1[n].float(), gp0[n].float(), rtol=5e-2,
                                   atol=2e-2 * float(gp0[n].float().abs().max()) + 1e-6, msg=n)


@pytest.mark.parametrize("premap", ["1", "0"])
def test_fused_premap_matches_separate_ops_on_cpu(cpu_kernels, monkeypatch, premap):
    """The block with K1 + K2 + K3 as one op (FLASH_MHC_FUSED_PREMAP=1) and as
    three ops (=0) gives identical outputs and parameter gradients, with and
    without activation checkpointing.  grad_x is the bf16 sum of x's three
    gradients (from K4, K3, K1): the separate ops let autograd add them as
    (g4 + g3) + g1, the pre-map op forms g4 + (g3 + g1), so the two may differ
    by a last bit of the sum."""
    from parity import check_chain

    def run(flag, ckpt):
        monkeypatch.setenv("FLASH_MHC_FUSED_PREMAP", flag)
        blk = _block(C=32)
        blk.activation_checkpointing = ckpt
        with torch.no_grad():
            blk.alpha_pre.fill_(0.8)
            blk.alpha_post.fill_(1.2)
            blk.alpha_res.fill_(1.7)
        x = rnd((64, 4, 32), 43).requires_grad_(True)
        out = blk._forward_triton(x)
        out.float().pow(2).sum().backward()
        return out.detach(), x.grad, {n: p.grad for n, p in blk.named_parameters()}

    ref = run("0", False)
    for ckpt in (False, True):
        o, gx, gp = run(premap, ckpt)
        assert torch.equal(o, ref[0])
        if premap == "0":
            assert torch.equal(gx, ref[1])
        else:
            check_chain("grad_x", gx.float(), ref[1].float(), max_rate=1.0)
        for n in gp:
            assert torch.equal(gp[n], ref[2][n]), n


@pytest.mark.parametrize("ckpt", [False, True])
def test_xgrad_sink_equals_autograd_sum_on_cpu(cpu_kernels, monkeypatch, ckpt):
    """Post-res's x-gradient sent through mhc_pre_map's x_sink and added in the
    pre-map backward (FLASH_MHC_FUSED_XGRAD=1) gives the same bits as leaving
    the sum to autograd (=0): both are bf16(g4 + bf16(pre-map gradient))."""

    def run(flag):
        monkeypatch.setenv("FLASH_MHC_FUSED_XGRAD", flag)
        blk = _block(C=32)
        blk.activation_checkpointing = ckpt
        with torch.no_grad():
            blk.alpha_pre.fill_(0.8)
            blk.alpha_post.fill_(1.2)
            blk.alpha_res.fill_(1.7)
        x = rnd((64, 4, 32), 47).requires_grad_(True)
        out = blk._forward_triton(x)
        out.float().pow(2).sum().backward()
        return out.detach(), x.grad, {n: p.grad for n, p in blk.named_parameters()}

    o1, gx1, gp1 = run("1")
    o0, gx0, gp0 = run("0")
    assert torch.equal(o1, o0)
    assert torch.equal(gx1, gx0)
    for n in gp0:
        assert torch.equal(gp1[n], gp0[n]), n


def test_pre_map_empty_batch_on_cpu(cpu_kernels):
    """T = 0 through the block's fused path: empty outputs and gradients (the
    sink of an empty batch has no storage to fill)."""
    blk = _block(C=32)
    x = rnd((0, 4, 32), 48).requires_grad_(True)
    out = blk._forward_triton(x)
    assert out.shape == (0, 4, 32)
    out.float().sum().backward()
    assert x.grad.shape == (0, 4, 32)
