"""The Qwen3.5 projection layout (qwowl35_amd/qwen35.py) against the 9B shapes
the reference runtime validates (qw35-server/src/model.rs:1563-1657) and
dispatches (Qw35MetalRuntime+Attention.m:35-37,113, +SSM.m:22-25,56,
+FFN.m:13-35): layer kinds, projection shapes, bytes per step, GEMV count."""
from __future__ import annotations


def test_layer_kinds_and_shapes():
    """Layer plan of the 9B: 24 delta and 8 attention layers, every 4th attention."""
    from qwowl35_amd import qwen35

    hp = qwen35.QWEN35_9B
    kinds = [qwen35.is_attention_layer(hp, il) for il in range(hp.transformer_layers)]
    assert sum(kinds) == 8 and [il for il, a in enumerate(kinds) if a] == [3, 7, 11, 15, 19, 23, 27, 31]
    shapes = {p.name: (p.rows, p.k) for p in qwen35.mixer_projections(hp, 0)}
    assert shapes == {"attn_qkv": (8192, 4096), "attn_gate": (4096, 4096), "ssm_beta": (32, 4096),
                      "ssm_alpha": (32, 4096), "ssm_out": (4096, 4096)}
    shapes = {p.name: (p.rows, p.k) for p in qwen35.mixer_projections(hp, 3)}
    assert shapes == {"attn_q": (8192, 4096), "attn_k": (1024, 4096), "attn_v": (1024, 4096),
                      "attn_output": (4096, 4096)}
    assert [(p.rows, p.k) for p in qwen35.ffn_projections(hp)] == [(12288, 4096), (12288, 4096), (4096, 12288)]
    assert qwen35.projection_bytes(hp, qwen35.StackTypes()) == 5_205_131_264
    assert qwen35.gemv_count(hp) == 217
