"""One Pairformer block on the HIP kernels.

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


@dataclass
class PairformerLayerWeights:
    """One Pairformer layer (Boltz-2 layout of sublayers), packed for the HIP
    kernels: the four triangle sublayers, the pair transition, the single
    attention with pair bias (with the layer's ``pre_norm_s``) and the single
    transition."""

    triangle: TriangleSublayers
    transition_z: kernels.TransitionWeights
    attention: kernels.SingleAttentionWeights
    transition_s: kernels.TransitionWeights

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor | None, pair_mask: torch.Tensor | None,
                eps: float = 1e-5) -> tuple[torch.Tensor, torch.Tensor]:
        """``B2K/pairformer.py:133-205``: z += tri-mul out, in, tri-attn start,
        end, transition; s += attention(LN(s), z, mask); s += transition_s.
        The attention's pair bias LN_z(z) w_z^T comes out of the pair
        transition's epilogue, so z is not read a further time."""
        z = self.triangle.forward(z, pair_mask)
        z, bias = kernels.transition(z, self.transition_z, residual=z, eps=eps, pair_bias_for=self.attention,
                                     pair_bias_eps=eps)
        s = kernels.single_attention(s, None, mask, self.attention, residual=s, eps=eps, pair_bias=bias)
        s = kernels.transition(s, self.transition_s, residual=s, eps=eps)
        return s, z

    @classmethod
    def from_fields(cls, w: dict, dtype: torch.dtype, device) -> "PairformerLayerWeights":
        """From torch-layout field dicts (``synthetic.pairformer_layer_weights``)."""
        return cls.from_boltz2(P.pairformer_layer_to_boltz2(w), dtype, device)

    @classmethod
    def from_boltz2(cls, p: dict, dtype: torch.dtype, device) -> "PairformerLayerWeights":
        """From a Boltz-2 layer dict (``M/boltz2/bridge/torch_mapping.py:603-650``)."""
        tri = TriangleSublayers(
            P.pack_trimul_boltz2(p["tri_mul_out"], dtype, device),
            P.pack_trimul_boltz2(p["tri_mul_in"], dtype, device),
            P.pack_triattn_boltz2(p["tri_att_start"], dtype, device),
            P.pack_triattn_boltz2(p["tri_att_end"], dtype, device),
        )
        return cls(
            triangle=tri,
            transition_z=P.pack_transition_boltz2(p["transition_z"], dtype, device),
            attention=P.pack_single_attention_boltz2(p["attention"], dtype, device, pre_norm=p["pre_norm_s"]),
            transition_s=P.pack_transition_boltz2(p["transition_s"], dtype, device),
        )

    @classmethod
    def random(cls, dtype: torch.dtype, device, seed: int = 2) -> "PairformerLayerWeights":
        return cls.from_fields(syn.pairformer_layer_weights(seed=seed), dtype, device)


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


def flops_block(n: int, c_z: int = 128, c_s: int = 384, heads_s: int = 16) -> dict[str, float]:
    """Algorithmic flops of one Pairformer layer, by sublayer."""
    tri = flops_triangle(n, c_z)
    single_attn = 2.0 * n * c_s * c_s * 5 + 4.0 * n * n * c_s + 2.0 * n * n * c_z * heads_s
    return {
        "trimul": 2 * tri["trimul"],
        "triattn": 2 * tri["triattn"],
        "transition_z": 24.0 * n * n * c_z * c_z,
        "single_attention": single_attn,
        "transition_s": 24.0 * n * c_s * c_s,
    }
