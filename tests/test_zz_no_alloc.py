"""GPU test of nerve_hip_fp8_output_projection_noalloc (the projection with
the library's static per-GPU scratch instead of its workspace): through the
C ABI, against nerve_hip_fp8_output_projection on the same inputs, bit for
bit, on two calls in a row (the second smaller), plus the refusal of a call
whose scratch would not fit."""
import numpy as np
import pytest

from nerve_amd import workloads as wl

from helpers import to_dev, to_np

pytestmark = pytest.mark.gpu


def _outputs(dev, M, N):
    import torch

    return (torch.full((M, N), float("nan"), dtype=torch.float32, device=dev),
            torch.full((M, N), 0x7FC0, dtype=torch.int16, device=dev),
            torch.full((M,), -1, dtype=torch.int32, device=dev))


def _run(ctx, dev, fn, d, spec):
    M, N = d["M"], d["N"]
    lf, lb, am = _outputs(dev, M, N)
    fn(spec, to_dev(d["x"], dev), to_dev(d["W"], dev), to_dev(d["scale_inv"], dev), lf, lb, am, M)
    return to_np(lf, np.float32), to_np(lb, np.uint16), to_np(am, np.uint32)


def test_noalloc_matches_workspace_entry_point(ctx, dev):
    # first call: the tiled form (M > 16); second, smaller: the M <= 16 stream form
    for seed, (M, N, K) in enumerate([(40, 4099, 2880), (3, 1000, 2880)]):
        rng = np.random.default_rng(700 + seed)
        d = wl.fp8_head(rng, N, K, M)
        spec = f"tied_output_projection_batch4_fp8_e4m3_b1x128_{N}x{K}_scale1_to_f32.comp"
        ref = _run(ctx, dev, ctx.fp8_output_projection, d, spec)
        got = _run(ctx, dev, ctx.fp8_output_projection_noalloc, d, spec)
        assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32)), (M, N, K)
        assert np.array_equal(got[1], ref[1]), (M, N, K)
        assert np.array_equal(got[2], ref[2]), (M, N, K)


def test_noalloc_refuses_oversized_scratch(ctx, dev):
    import torch

    from nerve_amd.hip import NerveHipError

    M, N, K = 512, 201088, 2880        # argmax partials alone need 6.4 MB
    spec = f"tied_output_projection_batch4_fp8_e4m3_b1x128_{N}x{K}_scale1_to_f32.comp"
    x = torch.zeros(M, K, dtype=torch.int16, device=dev)
    w = torch.zeros(16, dtype=torch.uint8, device=dev)       # never read: refused before any launch
    s = torch.zeros(16, dtype=torch.int16, device=dev)
    am = torch.zeros(M, dtype=torch.int32, device=dev)
    with pytest.raises(NerveHipError, match="static scratch"):
        ctx.fp8_output_projection_noalloc(spec, x, w, s, None, None, am, M)
