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
