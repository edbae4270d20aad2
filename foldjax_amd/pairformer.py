"""One Pairformer block's pair-track sublayers on the HIP kernels.

Order as in every port (``B2K/pairformer.py:133-172``,
``PXK/pairformer.py:49-140``, ``OF3/pair_block.py:106-190``): triangle
multiplication outgoing, incoming, triangle attention starting node, ending
node, each added to z as a residual (fused into the epilogue kernels).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from foldjax_amd import kernels
from foldjax_amd import params as P
from foldjax_amd import synthetic as syn


@dataclass
class TriangleSublayers:
    tri_mul_out: kernels.TriMulWeights
    tri_mul_in: kernels.TriMulWeights
    tri_att_start: kernels.TriAttnWeights
    tri_att_end: kernels.TriAttnWeights

    def forward(self, z: torch.Tensor, mask: torch.Tensor | None) -> torch.Tensor:
        z = kernels.trimul(z, mask, self.tri_mul_out, "outgoing", residual=z)
        z = kernels.trimul(z, mask, self.tri_mul_in, "incoming", residual=z)
        z = kernels.triattn(z, mask, self.tri_att_start, starting=True, residual=z)
        z = kernels.triattn(z, mask, self.tri_att_end, starting=False, residual=z)
        return z

    @classmethod
    def random(cls, dtype: torch.dtype, device, seed: int = 2, c_z: int = 128, heads: int = 4) -> "TriangleSublayers":
        tm = lambda s: P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(c_z, c_z, seed=s)), dtype, device)  # noqa: E731
        ta = lambda s: P.pack_triattn_protenix(  # noqa: E731
            P.triattn_to_protenix(syn.triattn_weights(c_z, heads, c_z // heads, seed=s)), dtype, device
        )
        return cls(tm(seed), tm(seed + 1), ta(seed + 2), ta(seed + 3))


def flops_triangle(n: int, c: int = 128, heads: int = 4, head_dim: int = 32) -> dict[str, float]:
    """Algorithmic flops per direction: the MFMA cores and the full sublayers."""
    contraction = 2.0 * n**3 * c
    attn_core = 4.0 * n**3 * heads * head_dim
    return {
        "contraction": contraction,
        "attn_core": attn_core,
        "trimul": contraction + 12.0 * n * n * c * c,
        "triattn": attn_core + n * n * c * (10.0 * heads * head_dim + 2.0 * heads),
    }
