"""Host harness checks that need no GPU: parameter count and state-dict names
match the reference model, the backend factory, and that the HIP path refuses
CPU tensors instead of falling back."""

import pytest
import torch

from model.config import ModelConfig
from model.model import SparDAResearchModel
from model.transformer import build_attention_backend


def test_parameter_count_matches_reference():
    # tests/test_model.py:9-29 of the reference: 102,451,968 with tied embeddings
    counts = SparDAResearchModel(ModelConfig()).count_parameters()
    assert counts["total"] == 102_451_968
    assert counts["embeddings"] == 32000 * 768


def test_state_dict_names_follow_the_reference_layout():
    sd = SparDAResearchModel(ModelConfig(n_layer=2)).state_dict()
    want = {"embeddings.weight", "final_norm.weight"}
    for i in range(2):
        p = f"layers.{i}."
        want |= {p + "attn_norm.weight", p + "ffn_norm.weight", p + "forecast.wf.weight",
                 p + "attention.wq.weight", p + "attention.wk.weight", p + "attention.wv.weight",
                 p + "attention.wo.weight", p + "ffn.w_gate.weight", p + "ffn.w_up.weight", p + "ffn.w_down.weight"}
    assert set(sd) == want


@pytest.mark.parametrize("name", ["dense", "sparse", "forecast", "static", "static_sparse", "offload",
                                  "async_offload", "hip_sparse", "hip_async_offload"])
def test_factory_builds_every_backend(name):
    cfg = ModelConfig(n_layer=1, attention_backend=name)
    attn = build_attention_backend(cfg, 1)
    assert {"wq", "wk", "wv", "wo"} <= set(dict(attn.named_children()))


def test_factory_rejects_unknown_backend():
    with pytest.raises(ValueError):
        build_attention_backend(ModelConfig(attention_backend="nope"), 0)


def test_hip_path_refuses_cpu_tensors():
    model = SparDAResearchModel(ModelConfig(n_layer=1, context_length=64)).eval()
    with torch.no_grad(), pytest.raises(RuntimeError, match="GPU"):
        model(torch.randint(0, 32000, (1, 16)))


def test_graph_decoder_refuses_cpu_models_and_unsupported_backends():
    from model.decode_graph import GraphDecoder
    cfg = ModelConfig(n_layer=2, context_length=1024)
    with pytest.raises(TypeError):
        GraphDecoder(SparDAResearchModel(cfg).to(torch.bfloat16), 1, 512)  # CPU weights: no fallback
    with pytest.raises(TypeError):
        GraphDecoder(SparDAResearchModel(cfg), 1, 512)  # fp32


def test_rope_known_answers():
    # tests/test_attention.py:11-21 of the reference: position 0 is the identity
    from model.rope import RotaryEmbedding, apply_rope, rope_tables
    cos, sin = rope_tables(64, 16)
    assert cos.shape == (16, 32) and sin.shape == (16, 32)
    assert torch.equal(cos[0], torch.ones(32)) and torch.equal(sin[0], torch.zeros(32))
    x = torch.randn(2, 1, 3, 64)
    assert torch.equal(apply_rope(x, cos, sin, offset=0), x)
    # rotate-half pairs (i, i + 32) at angle pos * 10000^(-2i/64)
    y = apply_rope(x, cos, sin, offset=5)
    ang = 5 * 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    c, s = torch.cos(ang), torch.sin(ang)
    a, b = x[..., :32].double(), x[..., 32:].double()
    want = torch.cat((a * c - b * s, b * c + a * s), dim=-1)
    assert torch.allclose(y.double(), want, atol=1e-5)
    rot = RotaryEmbedding(64, 16)
    q, k = rot(x, x[:, :, :1], offset=0)
    assert q.shape == x.shape and k.shape == (2, 1, 1, 64)
