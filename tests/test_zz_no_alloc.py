"""GPU test of fmhc_premap_fwd_noalloc, the pre-map forward that allocates
nothing (its few-token partial sums live in the library's static scratch
array): called through the C ABI, its outputs must equal fmhc_premap_fwd's
(the same kernels with a caller workspace) bit for bit, on consecutive calls
whose shapes shrink, so that the second call runs over what the first left in
the scratch."""

from __future__ import annotations

import pytest
import torch

from flash_mhc import _abi, build_permutation_matrices

pytestmark = pytest.mark.gpu

D = 32


def _inputs(T: int, C: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda")
    x = torch.randn(T, 4, C, generator=g).to(torch.bfloat16)
    x[:: max(1, T // 7)] *= 100  # rows far from unit RMS
    W = (torch.randn(D, 4 * C, generator=g) * 0.02).to(torch.bfloat16)
    alphas = [torch.tensor([a]) for a in (0.7, 0.4, 1.3)]
    bias = torch.randn(D, generator=g) * 0.5
    perm = build_permutation_matrices(4)[0]
    return [t.to(dev) for t in (x, W, *alphas, bias, perm)]


def _outputs(T: int, C: int, with_li: bool):
    dev = torch.device("cuda")
    f32 = torch.float32
    li = torch.full((T, C), -1, dtype=torch.int16, device=dev).view(torch.bfloat16) if with_li else None
    return dict(li=li, proj=torch.full((T, D), -1, dtype=torch.int16, device=dev).view(torch.bfloat16),
                inv=torch.full((T,), float("nan"), device=dev), h_pre=torch.full((T, 4), float("nan"), device=dev),
                h_post=torch.full((T, 4), float("nan"), device=dev),
                H=torch.full((T, 4, 4), float("nan"), device=dev, dtype=f32))


def _call(noalloc: bool, T: int, C: int, inp, out):
    lib = _abi.load()
    x, W, ap, apo, ar, b, perm = inp
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    head = (x.data_ptr(), W.data_ptr(), ap.data_ptr(), apo.data_ptr(), ar.data_ptr(), b.data_ptr(),
            perm.data_ptr(), 0, ptr(out["li"]), out["proj"].data_ptr(), out["inv"].data_ptr(),
            out["h_pre"].data_ptr(), out["h_post"].data_ptr(), out["H"].data_ptr(), None, None)
    if noalloc:
        status = lib.fmhc_premap_fwd_noalloc(*head, T, C, 4, st)
    else:
        nbytes = int(lib.fmhc_premap_fwd_workspace_bytes(T, C))
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device="cuda")
        status = lib.fmhc_premap_fwd(*head, ws.data_ptr(), nbytes, T, C, 4, st)
        torch.cuda.synchronize()  # ws stays alive until the kernels have run
    _abi.check(status, "premap_fwd_noalloc" if noalloc else "premap_fwd")


def _same(a: torch.Tensor | None, b: torch.Tensor | None, what: str) -> None:
    if a is None:
        assert b is None
        return
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32)), what


# Shrinking shapes in a row.  (2032, 320) needs the largest scratch of any
# shape (2,145,792 bytes); (100, 1024) and (1, 4096) take fewer column splits
# over the same array; (4096, 256) takes no scratch (one-pass forward).
SEQUENCE = [(2032, 320, True), (100, 1024, True), (1, 4096, False), (4096, 256, True), (33, 1000, True)]


def _run_sequence(order):
    lib = _abi.load()
    for i, (T, C, with_li) in enumerate(order):
        print(f"[no-alloc] call {i}: T={T} C={C} layer_input={with_li}", flush=True)
        inp = _inputs(T, C, seed=10 + i)
        got, want = _outputs(T, C, with_li), _outputs(T, C, with_li)
        _call(True, T, C, inp, got)
        _call(False, T, C, inp, want)
        torch.cuda.synchronize()
        for k in want:
            _same(got[k], want[k], f"call {i} (T={T}, C={C}): {k}")
        need = int(lib.fmhc_premap_fwd_workspace_bytes(T, C))
        assert need <= 4 << 20


def test_noalloc_matches_workspace_entry_point():
    _run_sequence(SEQUENCE)


def test_noalloc_two_calls_second_smaller():
    # The minimal sequence: a large split, then a smaller input over the same scratch.
    _run_sequence([(1024, 1024, True), (17, 1024, True)])


def test_noalloc_rejects_bad_arguments_and_empty_batch():
    lib = _abi.load()
    st = torch.cuda.current_stream().cuda_stream
    args = [None] * 7 + [0] + [None] * 8
    assert lib.fmhc_premap_fwd_noalloc(*args, -1, 16, 4, st) == 1  # T < 0
    assert lib.fmhc_premap_fwd_noalloc(*args, 8, 16, 3, st) == 1  # n != 4
    assert lib.fmhc_premap_fwd_noalloc(*args, 0, 16, 4, st) == 0  # empty batch: nothing to do
    assert b"scratch" in lib.fmhc_error_string(2)
