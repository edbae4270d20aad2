"""Field dicts of the Protenix and OpenFold3 containers for the oracle, built
from the torch-layout synthetic weights (``foldjax_amd.synthetic``): the
oracle reads the reference's field names from plain dicts."""

from __future__ import annotations


def of3_attn(p):
    return {"layer_norm": p["layer_norm"], "linear_z": p["linear"], "mha": p["attention"]}


def px_apb_fields(p):
    """Protenix ``AttentionPairBiasParams`` fields from a torch-layout
    single-attention dict (``synthetic.single_attention_weights``)."""
    return {
        "layernorm_a": p["pre_norm_s"],
        "attention": {"linear_q": p["proj_q"], "linear_k": p["proj_k"], "linear_v": p["proj_v"],
                      "linear_o": p["proj_o"], "linear_g": p["proj_g"]},
        "layernorm_z": p["proj_z_norm"],
        "linear_z": p["proj_z"],
    }


def of3_apb_fields(p):
    px = px_apb_fields(p)
    return {"layer_norm_a": px["layernorm_a"], "layer_norm_z": px["layernorm_z"], "linear_z": px["linear_z"],
            "mha": px["attention"]}


def px_block_fields(w):
    return {
        "tri_mul_out": w["tri_mul_out"], "tri_mul_in": w["tri_mul_in"],
        "tri_att_start": w["tri_att_start"], "tri_att_end": w["tri_att_end"],
        "pair_transition": w["transition_z"],
        "attention_pair_bias": px_apb_fields(w["attention"]),
        "single_transition": w["transition_s"],
    }


def of3_block_fields(w):
    return {
        "pair_stack": {"tri_mul_out": w["tri_mul_out"], "tri_mul_in": w["tri_mul_in"],
                       "tri_att_start": of3_attn(w["tri_att_start"]), "tri_att_end": of3_attn(w["tri_att_end"]),
                       "pair_transition": w["transition_z"]},
        "attn_pair_bias": of3_apb_fields(w["attention"]),
        "single_transition": w["transition_s"],
    }
