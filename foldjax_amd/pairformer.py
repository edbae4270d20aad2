"""One Pairformer block on the HIP kernels.

Order as in every port (``B2K/pairformer.py:133-172``,
``PXK/pairformer.py:49-140``, ``OF3/pair_block.py:106-190``): triangle
multiplication outgoing, incoming, triangle attention starting node, ending
node, pair transition, each added to z as a residual (fused into the
epilogue kernels); then the single track's attention with pair bias and
transition.
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

    def forward(self, z: torch.Tensor, mask: torch.Tensor | None, *, inf: float = 1e9, eps: float = 1e-5,
                out_mask: torch.Tensor | None = None, tri_mul_first: bool = True,
                donate: bool = False) -> torch.Tensor:
        """z += each sublayer in turn (the residual fused into its epilogue);
        with ``out_mask`` every sublayer's output is multiplied by
        ``out_mask != 0`` (Protenix's ``z * pair_gate``). ``tri_mul_first``
        orders the multiplication pair before the attention pair (OpenFold3's
        ``pair_block`` option).

        The sublayers update one pair tensor in place: the first writes a new
        tensor and the others overwrite it (the kernels read each position's
        inputs before writing it), so the four sublayers allocate one pair
        tensor. ``donate``: the caller gives up ``z`` (a contiguous tensor it
        no longer reads, as the reference's scan donates its carry,
        ``B2K/pairformer.py:74-96``), and the first sublayer overwrites it as
        well."""
        first = [True]

        def dest(z):
            # the output buffer of the next sublayer: z itself, except for the
            # first sublayer of a call that does not donate z
            if first[0]:
                first[0] = False
                return z if donate and z.is_contiguous() else None
            return z

        def mul_pair(z):
            z = kernels.trimul(z, mask, self.tri_mul_out, "outgoing", eps=eps, residual=z, out_mask=out_mask,
                               out=dest(z))
            return kernels.trimul(z, mask, self.tri_mul_in, "incoming", eps=eps, residual=z, out_mask=out_mask,
                                  out=dest(z))

        def att_pair(z):
            z = kernels.triattn(z, mask, self.tri_att_start, starting=True, inf=inf, eps=eps, residual=z,
                                out_mask=out_mask, out=dest(z))
            return kernels.triattn(z, mask, self.tri_att_end, starting=False, inf=inf, eps=eps, residual=z,
                                   out_mask=out_mask, out=dest(z))

        return att_pair(mul_pair(z)) if tri_mul_first else mul_pair(att_pair(z))

    @classmethod
    def random(cls, dtype: torch.dtype, device, seed: int = 2, c_z: int = 128, heads: int = 4) -> "TriangleSublayers":
        tm = lambda s: P.pack_trimul_torch(P.trimul_to_protenix(syn.trimul_weights(c_z, c_z, seed=s)), dtype, device)  # noqa: E731
        ta = lambda s: P.pack_triattn_protenix(  # noqa: E731
            P.triattn_to_protenix(syn.triattn_weights(c_z, heads, c_z // heads, seed=s)), dtype, device
        )
        return cls(tm(seed), tm(seed + 1), ta(seed + 2), ta(seed + 3))


def _same(t: torch.Tensor | None, u: torch.Tensor) -> bool:
    return t is not None and t.dtype == u.dtype


@dataclass
class PairformerLayerWeights:
    """One Pairformer block packed for the HIP kernels: the four triangle
    sublayers, the pair transition, and (when the block has a single track)
    the single attention with pair bias and the single transition. The single
    track may be packed in another dtype than the pair track (Boltz-2 runs it
    in float32 over a bfloat16 pair tensor). One packed object serves every
    port; the port's block function picks the forward below."""

    triangle: TriangleSublayers
    transition_z: kernels.TransitionWeights
    attention: kernels.SingleAttentionWeights | None
    transition_s: kernels.TransitionWeights | None

    def _pair_bias_prep(self, s: torch.Tensor | None, z: torch.Tensor):
        """The attention whose pair bias the pair transition emits: a single
        track in the pair track's dtype, or a float32 one over a bfloat16
        pair track (the bias then comes out in float32)."""
        if self.attention is None or s is None or not _same(self.attention.q_weight, s):
            return None
        if s.dtype == z.dtype or (s.dtype == torch.float32 and z.dtype == torch.bfloat16):
            return self.attention
        return None

    def _pair_transition(self, z, s, *, row_mask=None, out_mask=None, eps=1e-5):
        """z += transition(z) in place (z is the triangle sublayers' own
        output), with the single attention's pair bias when it applies."""
        att = self._pair_bias_prep(s, z)
        if att is None:
            return kernels.transition(z, self.transition_z, row_mask=row_mask, residual=z, eps=eps,
                                      out_mask=out_mask, out=z), None
        return kernels.transition(z, self.transition_z, row_mask=row_mask, residual=z, eps=eps, out_mask=out_mask,
                                  pair_bias_for=att, pair_bias_eps=eps, out=z)

    @staticmethod
    def _s_dest(s, donate):
        return s if donate and s is not None and s.is_contiguous() else None

    def forward(self, s: torch.Tensor, z: torch.Tensor, mask: torch.Tensor | None, pair_mask: torch.Tensor | None,
                eps: float = 1e-5, *, donate: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """Boltz-2 ``pairformer_layer_forward`` (``B2K/pairformer.py:133-205``):
        z += tri-mul out, in, tri-attn start, end, transition; s +=
        attention(LN(s), z, mask); s += transition_s. The attention's pair
        bias LN_z(z) w_z^T comes out of the pair transition's epilogue (in
        float32 when s is float32 over a bfloat16 z), so z is not read a
        further time. The block allocates one pair tensor and one single
        tensor for its outputs and updates them in place; with ``donate`` it
        allocates neither and overwrites s and z (``TriangleSublayers.forward``)."""
        z = self.triangle.forward(z, pair_mask, eps=eps, donate=donate)
        z, bias = self._pair_transition(z, s, eps=eps)
        s = kernels.single_attention(s, None if bias is not None else z, mask, self.attention, residual=s, eps=eps,
                                     pair_bias=bias, out=self._s_dest(s, donate))
        s = kernels.transition(s, self.transition_s, residual=s, eps=eps, out=s)
        return s, z

    def forward_protenix(self, s: torch.Tensor | None, z: torch.Tensor,
                         pair_mask: torch.Tensor | None, *, donate: bool = False
                         ) -> tuple[torch.Tensor | None, torch.Tensor]:
        """Protenix ``pairformer_block`` (``PXK/pairformer.py:49-180``). Every
        sublayer's output is multiplied by ``pair_gate = bool(pair_mask)``
        inside its epilogue. Gating z (and s) on entry as well is not needed
        for finite inputs: a gated position enters the next sublayer only
        where the pair mask already zeroes its contribution, and the first
        output gate zeroes it. ``single_valid`` (the boolean diagonal of the
        pair mask) is the single attention's key mask with ``inf = 1e10`` and
        gates its output and the single transition's; the reference's extra
        bias ``-1e10`` on invalid query rows changes only rows that the gate
        then zeroes. ``donate`` as for ``forward``."""
        valid = None
        if pair_mask is not None:
            valid = torch.diagonal(pair_mask, dim1=-2, dim2=-1).ne(0)
        z = self.triangle.forward(z, pair_mask, out_mask=pair_mask, donate=donate)
        z, bias = self._pair_transition(z, s, out_mask=pair_mask)
        if self.attention is None:
            if s is not None and valid is not None:
                s = s * valid.to(s.dtype)[..., None]
            return s, z
        if s is None:
            raise ValueError("PairformerBlock single path requires s")
        if self.transition_s is None:
            raise ValueError("missing single_transition for single path")
        s = kernels.single_attention(s, None if bias is not None else z, valid, self.attention, inf=1e10,
                                     residual=s, pair_bias=bias, out_mask=valid, out=self._s_dest(s, donate))
        s = kernels.transition(s, self.transition_s, residual=s, out_mask=valid, out=s)
        return s, z

    def forward_openfold3(self, s: torch.Tensor, z: torch.Tensor, single_mask: torch.Tensor | None,
                          pair_mask: torch.Tensor | None, *, inf: float = 1e9, mask_transition: bool = True,
                          eps: float = 1e-5, donate: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """OpenFold3 ``pairformer_block`` (``OF3/pairformer.py:42-102``): the
        pair block (``OF3/pair_block.py:106-190``), then s += attention with
        pair bias (key mask ``single_mask``, ``inf``) and the SwiGLU single
        transition, whose update is multiplied by ``single_mask`` when
        ``mask_transition``. ``donate`` as for ``forward``."""
        z = self.triangle.forward(z, pair_mask, inf=inf, eps=eps, donate=donate)
        z, bias = self._pair_transition(z, s, row_mask=pair_mask if mask_transition else None, eps=eps)
        s = kernels.single_attention(s, None if bias is not None else z, single_mask, self.attention, inf=inf,
                                     eps=eps, residual=s, pair_bias=bias, out=self._s_dest(s, donate))
        s = kernels.transition(s, self.transition_s, row_mask=single_mask if mask_transition else None, residual=s,
                               eps=eps, out=s)
        return s, z

    @classmethod
    def from_fields(cls, w: dict, dtype: torch.dtype, device, single_dtype: torch.dtype | None = None
                    ) -> "PairformerLayerWeights":
        """From torch-layout field dicts (``synthetic.pairformer_layer_weights``)."""
        return cls.from_boltz2(P.pairformer_layer_to_boltz2(w), dtype, device, single_dtype=single_dtype)

    @classmethod
    def from_boltz2(cls, p: dict, dtype: torch.dtype, device, single_dtype: torch.dtype | None = None
                    ) -> "PairformerLayerWeights":
        """From a Boltz-2 layer dict (``M/boltz2/bridge/torch_mapping.py:603-650``);
        the single track in ``single_dtype`` (default: ``dtype``)."""
        sd = dtype if single_dtype is None else single_dtype
        tri = TriangleSublayers(
            P.pack_trimul_boltz2(p["tri_mul_out"], dtype, device),
            P.pack_trimul_boltz2(p["tri_mul_in"], dtype, device),
            P.pack_triattn_boltz2(p["tri_att_start"], dtype, device),
            P.pack_triattn_boltz2(p["tri_att_end"], dtype, device),
        )
        return cls(
            triangle=tri,
            transition_z=P.pack_transition_boltz2(p["transition_z"], dtype, device),
            attention=P.pack_single_attention_boltz2(p["attention"], sd, device, pre_norm=p["pre_norm_s"]),
            transition_s=P.pack_transition_boltz2(p["transition_s"], sd, device),
        )

    @classmethod
    def from_protenix(cls, p, dtype: torch.dtype, device, single_dtype: torch.dtype | None = None
                      ) -> "PairformerLayerWeights":
        """From a Protenix ``PairformerBlockParams`` (``PXK/pairformer.py:31-41``);
        fields may already be packed weight objects."""
        sd = dtype if single_dtype is None else single_dtype

        def pk(obj, packer, kind, dt):
            return obj if isinstance(obj, kind) else packer(obj, dt, device)

        tri = TriangleSublayers(
            pk(p.tri_mul_out, P.pack_trimul_torch, kernels.TriMulWeights, dtype),
            pk(p.tri_mul_in, P.pack_trimul_torch, kernels.TriMulWeights, dtype),
            pk(p.tri_att_start, P.pack_triattn_protenix, kernels.TriAttnWeights, dtype),
            pk(p.tri_att_end, P.pack_triattn_protenix, kernels.TriAttnWeights, dtype),
        )
        apb, st = p.attention_pair_bias, p.single_transition
        return cls(
            triangle=tri,
            transition_z=pk(p.pair_transition, P.pack_transition_torch, kernels.TransitionWeights, dtype),
            attention=None if apb is None else pk(apb, P.pack_single_attention_protenix,
                                                  kernels.SingleAttentionWeights, sd),
            transition_s=None if st is None else pk(st, P.pack_transition_torch, kernels.TransitionWeights, sd),
        )

    @classmethod
    def from_openfold3(cls, p, dtype: torch.dtype, device, single_dtype: torch.dtype | None = None
                       ) -> "PairformerLayerWeights":
        """From an OpenFold3 ``PairformerBlockParams`` (``OF3/pairformer.py:27-33``)."""
        sd = dtype if single_dtype is None else single_dtype

        def pk(obj, packer, kind, dt):
            return obj if isinstance(obj, kind) else packer(obj, dt, device)

        ps = p.pair_stack
        tri = TriangleSublayers(
            pk(ps.tri_mul_out, P.pack_trimul_torch, kernels.TriMulWeights, dtype),
            pk(ps.tri_mul_in, P.pack_trimul_torch, kernels.TriMulWeights, dtype),
            pk(ps.tri_att_start, P.pack_triattn_openfold3, kernels.TriAttnWeights, dtype),
            pk(ps.tri_att_end, P.pack_triattn_openfold3, kernels.TriAttnWeights, dtype),
        )
        return cls(
            triangle=tri,
            transition_z=pk(ps.pair_transition, P.pack_transition_openfold3, kernels.TransitionWeights, dtype),
            attention=pk(p.attn_pair_bias, P.pack_single_attention_openfold3, kernels.SingleAttentionWeights, sd),
            transition_s=pk(p.single_transition, P.pack_transition_openfold3, kernels.TransitionWeights, sd),
        )

    @classmethod
    def random(cls, dtype: torch.dtype, device, seed: int = 2, single_dtype: torch.dtype | None = None
               ) -> "PairformerLayerWeights":
        return cls.from_fields(syn.pairformer_layer_weights(seed=seed), dtype, device, single_dtype=single_dtype)


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
