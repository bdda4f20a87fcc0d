"""Write tests/golden/block_fallback_n4_C16.safetensors from the reference.

What it pins (nothing in the math checks does): the reference's MHCLiteBlock
(alint77/flash-mHC src/flash_mhc/block.py) construction under a fixed seed --
parameter registration order, hence state_dict keys/order and initial values --
and the end-to-end output and gradients of its plain-PyTorch path
(_forward_pytorch, block.py:126-148) in fp32 on the CPU, with and without
activation checkpointing.

Run where the reference is mounted (it never ships with this repository):
    python tests/golden/make_block_golden.py /root/reference
The output holds data only: inputs, parameters and expected values.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
OUT = HERE / "block_fallback_n4_C16.safetensors"

T, N, C = 8, 4, 16
SEED = 0


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    from flash_mhc.block import MHCLiteBlock  # the reference's module

    torch.manual_seed(SEED)
    layer = torch.nn.Sequential(torch.nn.Linear(C, C, bias=False), torch.nn.GELU())
    blk = MHCLiteBlock(N, C, layer, triton_fused=False)
    keys = list(blk.state_dict().keys())
    tensors = {f"state.{k}": v.detach().clone().contiguous() for k, v in blk.state_dict().items()}

    g = torch.Generator().manual_seed(SEED + 1)
    x = torch.randn(T, N, C, generator=g)
    tensors["x"] = x.clone()
    for ckpt in (False, True):
        blk.activation_checkpointing = ckpt
        blk.zero_grad()
        xi = x.clone().requires_grad_(True)
        out = blk._forward_pytorch(xi)
        (out * out).sum().backward()
        tag = "ckpt" if ckpt else "plain"
        tensors[f"{tag}.out"] = out.detach().clone()
        tensors[f"{tag}.grad.x"] = xi.grad.detach().clone()
        for name, p in blk.named_parameters():
            tensors[f"{tag}.grad.{name}"] = p.grad.detach().clone().contiguous()
    meta = {"state_dict_keys": json.dumps(keys), "T": str(T), "n": str(N), "C": str(C),
            "seed": str(SEED), "loss": "sum(out**2)",
            "layer": "Sequential(Linear(C, C, bias=False), GELU())",
            "torch": torch.__version__}
    save_file(tensors, str(OUT), metadata=meta)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes), keys={keys}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
