"""CPU tests of the MHCLiteBlock API and of its plain-PyTorch path.

The golden fixture (tests/golden/block_fallback_n4_C16.safetensors, written by
tests/golden/make_block_golden.py from the reference's own block) pins the
constructor (registration order -> state_dict keys and seeded initial values)
and the plain path's outputs and gradients, with and without activation
checkpointing.  The oracle's block formula is pinned against the same data.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

import flash_mhc
from flash_mhc import MHCLiteBlock
from oracle import mhc_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "block_fallback_n4_C16.safetensors"


def golden():
    tensors = load_file(str(GOLDEN))
    with safe_open(str(GOLDEN), "pt") as f:
        meta = f.metadata()
    return tensors, meta


def make_block(C=16, seed=0):
    torch.manual_seed(seed)
    layer = torch.nn.Sequential(torch.nn.Linear(C, C, bias=False), torch.nn.GELU())
    return MHCLiteBlock(4, C, layer, triton_fused=False)


def test_state_dict_and_init_match_reference():
    t, meta = golden()
    blk = make_block()
    keys = json.loads(meta["state_dict_keys"])
    assert list(blk.state_dict().keys()) == keys
    for k, v in blk.state_dict().items():
        assert torch.equal(v, t[f"state.{k}"]), k


def test_reference_state_dict_loads_strictly():
    t, _ = golden()
    sd = {k[len("state."):]: v for k, v in t.items() if k.startswith("state.")}
    blk = make_block(seed=123)
    blk.load_state_dict(sd, strict=True)
    for k, v in blk.state_dict().items():
        assert torch.equal(v, sd[k])


@pytest.mark.parametrize("tag", ["plain", "ckpt"])
def test_plain_path_matches_reference_fixture(tag):
    t, _ = golden()
    blk = make_block()
    blk.activation_checkpointing = tag == "ckpt"
    x = t["x"].clone().requires_grad_(True)
    out = blk._forward_pytorch(x)
    (out * out).sum().backward()
    torch.testing.assert_close(out, t[f"{tag}.out"], rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(x.grad, t[f"{tag}.grad.x"], rtol=1e-5, atol=1e-6)
    for name, p in blk.named_parameters():
        torch.testing.assert_close(p.grad, t[f"{tag}.grad.{name}"], rtol=1e-5, atol=1e-6, msg=name)


def test_oracle_block_matches_reference_fixture():
    t, _ = golden()
    params = {
        "W": t["state.W_all.weight"], "b": t["state.W_all.bias"],
        "alpha_pre": t["state.alpha_pre"], "alpha_post": t["state.alpha_post"],
        "alpha_res": t["state.alpha_res"], "perm": O.permutation_matrices(4)[0],
    }
    assert torch.equal(params["perm"], t["state.perm_mat"])
    lin = torch.nn.Linear(16, 16, bias=False)
    lin.weight.data.copy_(t["state.layer.0.weight"])
    layer = torch.nn.Sequential(lin, torch.nn.GELU())
    out = O.block_forward(t["x"], params, layer, 4)
    torch.testing.assert_close(out, t["plain.out"], rtol=1e-6, atol=1e-6)


def test_constructor_surface():
    blk = MHCLiteBlock(4, 32, torch.nn.Identity(), triton_fused=True, activation_checkpointing=True)
    assert (blk.n, blk.C, blk.nC, blk.n_fact, blk.identity_idx) == (4, 32, 128, 24, 0)
    assert blk.triton_fused and blk.activation_checkpointing
    assert blk.W_all.weight.shape == (32, 128) and blk.W_all.bias.shape == (32,)
    for a in (blk.alpha_pre, blk.alpha_post, blk.alpha_res):
        assert a.shape == (1,) and float(a.detach()) == pytest.approx(0.01)
    assert blk.perm_mat.shape == (24, 16)
    assert [n for n, _ in blk.named_parameters()] == ["alpha_pre", "alpha_post", "alpha_res", "W_all.weight", "W_all.bias"]
    assert hasattr(blk, "_forward_pytorch") and hasattr(blk, "_forward_triton")
    assert set(flash_mhc.__all__) == {"MHCLiteBlock", "build_permutation_matrices"}


def test_cpu_input_takes_plain_path(monkeypatch):
    blk = make_block()

    def boom(*a, **k):
        raise AssertionError("fused path must not run for CPU tensors")

    monkeypatch.setattr(blk, "_forward_triton", boom)
    out = blk(torch.randn(4, 4, 16))
    assert out.shape == (4, 4, 16)


def test_private_torch_queries_fall_back(monkeypatch):
    """The eager fast paths rely on two private torch queries; a torch build
    without them must still import the package and make _plain_eager False
    (the torch.library ops then run), not raise."""
    from flash_mhc import block as B

    assert B._private_probe(lambda: torch._C._no_such_query_in_torch) is None

    def missing():
        from torch.utils._python_dispatch import _no_such_function  # noqa: F401

    assert B._private_probe(missing) is None
    x = torch.empty(1)
    monkeypatch.setattr(B, "_dispatch_mode", None)
    assert B._plain_eager(x) is False
    monkeypatch.setattr(B, "_functorch_active", None)
    assert B._plain_eager(x) is False


def test_kwargs_reach_the_layer():
    class L(torch.nn.Module):
        def forward(self, x, *, scale=1.0):
            return x * scale

    blk = MHCLiteBlock(4, 8, L(), triton_fused=False)
    x = torch.randn(3, 4, 8)
    a = blk(x, scale=2.0)
    b = blk(x, scale=0.0)
    assert not torch.allclose(a, b)


@pytest.mark.parametrize("n", [2, 3, 4])
def test_plain_path_other_n_and_leading_dims(n):
    torch.manual_seed(0)
    C = 6
    blk = MHCLiteBlock(n, C, torch.nn.Linear(C, C, bias=False)).double()
    x = torch.randn(2, 5, n, C, dtype=torch.float64)
    out = blk(x)
    assert out.shape == x.shape
    params = {"W": blk.W_all.weight, "b": blk.W_all.bias, "alpha_pre": blk.alpha_pre,
              "alpha_post": blk.alpha_post, "alpha_res": blk.alpha_res,
              "perm": O.permutation_matrices(n)[0]}
    ref = O.block_forward(x, params, blk.layer, n)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    assert blk.n_fact == math.factorial(n)


def test_checkpointing_predicate():
    blk = make_block()
    blk.activation_checkpointing = True
    x = torch.randn(2, 4, 16, requires_grad=True)
    assert blk._use_activation_checkpointing(x)
    blk.eval()
    assert not blk._use_activation_checkpointing(x)
    blk.train()
    with torch.no_grad():
        assert not blk._use_activation_checkpointing(x)
    assert not blk._use_activation_checkpointing(x.detach())


def test_rmsnorm_weight_option():
    torch.manual_seed(0)
    C = 8
    plain = MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False))
    torch.manual_seed(0)
    blk = MHCLiteBlock(4, C, torch.nn.Linear(C, C, bias=False), rmsnorm_weight=True).double()
    assert "rms_weight" not in plain.state_dict() and plain.rms_weight is None
    assert list(blk.state_dict())[:4] == ["alpha_pre", "alpha_post", "alpha_res", "rms_weight"]
    with torch.no_grad():
        blk.rms_weight.copy_(1 + 0.1 * torch.randn(4 * C, dtype=torch.float64))
    x = torch.randn(5, 4, C, dtype=torch.float64, requires_grad=True)
    out = blk(x)
    # rmsnorm(x) * g @ W^T == rmsnorm(x) @ (W * g)^T
    params = {"W": blk.W_all.weight * blk.rms_weight, "b": blk.W_all.bias, "alpha_pre": blk.alpha_pre,
              "alpha_post": blk.alpha_post, "alpha_res": blk.alpha_res, "perm": O.permutation_matrices(4)[0]}
    torch.testing.assert_close(out, O.block_forward(x, params, blk.layer, 4), rtol=1e-12, atol=1e-12)
    out.sum().backward()
    assert blk.rms_weight.grad is not None and torch.isfinite(blk.rms_weight.grad).all()
