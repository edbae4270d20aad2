"""The allocation-free tri-mul entry point (``fjx_trimul_fwd_noalloc``) against
``fjx_trimul_fwd``, through the C ABI.

Both run the same kernels on the same inputs, one with a caller workspace and
one on the library's static per-GPU scratch, so their outputs must be
bit-identical. Two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents), cover both contraction kernels
(n a multiple of 256: the LDS-DMA kernel; otherwise the register-staged one)
and both dtypes. A shape whose workspace exceeds the scratch is refused on
the host before anything is launched.
"""

from __future__ import annotations

import pytest
import torch

from foldjax_amd import _lib, kernels
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _case(n, dtype, seed):
    z = torch.from_numpy(syn.pair_input(n, 128, seed=seed)).to("cuda", dtype)
    m = torch.from_numpy(syn.pair_mask(n, n - n // 10)).to("cuda", dtype)
    w = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(seed=seed + 1)), dtype, "cuda")
    return z, m, w


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry(dt):
    for n, direction, seed in ((256, "outgoing", 3), (100, "incoming", 5)):
        say(f"noalloc trimul n={n} {direction} {dt}")
        z, m, w = _case(n, dt, seed)
        want = kernels.trimul(z, m, w, direction, residual=z)
        got = kernels.trimul(z, m, w, direction, residual=z, no_alloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), f"n={n} {direction}: noalloc output differs from fjx_trimul_fwd"


def test_noalloc_refuses_shapes_beyond_scratch():
    say("noalloc trimul refusal n=600")
    n = 600  # bf16 workspace 3 * 600^2 * 128 * 2 B = 276 MB > 256 MiB
    lib = _lib.load()
    assert lib.fjx_trimul_workspace_size(1, n, 128, 128, _lib.FJX_DTYPE_BF16) > _lib.NOALLOC_SCRATCH_BYTES
    z = torch.zeros((n, n, 128), device="cuda", dtype=torch.bfloat16)
    w = P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(seed=1)), torch.bfloat16, "cuda")
    with pytest.raises(_lib.FjxError, match="static scratch holds"):
        kernels.trimul(z, None, w, "outgoing", no_alloc=True)
    # the largest bf16 shape that fits runs, close to the scratch's end, and
    # matches the workspace entry bit for bit
    n_fit = 591
    assert lib.fjx_trimul_workspace_size(1, n_fit, 128, 128, _lib.FJX_DTYPE_BF16) <= _lib.NOALLOC_SCRATCH_BYTES
    assert lib.fjx_trimul_workspace_size(1, n_fit + 1, 128, 128, _lib.FJX_DTYPE_BF16) > _lib.NOALLOC_SCRATCH_BYTES
    say(f"noalloc trimul at the scratch limit n={n_fit}")
    z, m, w = _case(n_fit, torch.bfloat16, 7)
    want = kernels.trimul(z, m, w, "incoming", residual=z)
    got = kernels.trimul(z, m, w, "incoming", residual=z, no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"n={n_fit}: noalloc output differs from fjx_trimul_fwd"
