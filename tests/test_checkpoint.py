"""Checkpoint loading on the CPU: load_skeleton (the reference's model.py:20-55) and
load_skeleton_gptoss (gptoss.py:146-176) on small transformers models written as safetensors
checkpoints, sharded with an index (as published) and as one file. Every non-expert tensor
and gpt-oss expert bias must arrive unchanged; the expert tensors stay out of the model."""

import json
import os

import pytest
import torch

transformers = pytest.importorskip("transformers")
safetensors_torch = pytest.importorskip("safetensors.torch")

from wisp.gptoss import PagedGptOssBlock  # noqa: E402
from wisp.model import load_skeleton  # noqa: E402
from wisp.moe import PagedMoEBlock, Runtime  # noqa: E402
from wisp.store import SafetensorsDir  # noqa: E402


def write_checkpoint(path, cfg, tensors, sharded):
    """config.json + the tensors as model.safetensors, or as two shards with an index."""
    os.makedirs(path, exist_ok=True)
    cfg.save_pretrained(path)
    tensors = {k: v.detach().contiguous().clone() for k, v in tensors.items()}
    if not sharded:
        safetensors_torch.save_file(tensors, os.path.join(path, "model.safetensors"))
        return
    names = sorted(tensors)
    files = {"model-00001-of-00002.safetensors": names[::2], "model-00002-of-00002.safetensors": names[1::2]}
    weight_map = {}
    for f, part in files.items():
        safetensors_torch.save_file({k: tensors[k] for k in part}, os.path.join(path, f))
        weight_map.update({k: f for k in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {}, "weight_map": weight_map}, fh)


def qwen3_checkpoint_tensors(model, per_expert=True):
    """The model's state dict with its fused expert tensors written per expert, as the
    published Qwen3-MoE checkpoints name them (or kept fused)."""
    out = {k: v for k, v in model.state_dict().items() if ".mlp.experts." not in k}
    I = model.config.moe_intermediate_size
    for l, lay in enumerate(model.model.layers):
        ex, p = lay.mlp.experts, f"model.layers.{l}.mlp.experts."
        if not per_expert:
            out[p + "gate_up_proj"], out[p + "down_proj"] = ex.gate_up_proj, ex.down_proj
            continue
        for e in range(ex.gate_up_proj.shape[0]):
            out[f"{p}{e}.gate_proj.weight"] = ex.gate_up_proj[e, :I]
            out[f"{p}{e}.up_proj.weight"] = ex.gate_up_proj[e, I:]
            out[f"{p}{e}.down_proj.weight"] = ex.down_proj[e]
    return out


def tiny_qwen3(seed=0):
    torch.manual_seed(seed)
    cfg = transformers.Qwen3MoeConfig(vocab_size=96, hidden_size=64, intermediate_size=96, moe_intermediate_size=32,
                                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                                      num_experts=4, num_experts_per_tok=2, norm_topk_prob=True,
                                      max_position_embeddings=128, decoder_sparse_step=1, mlp_only_layers=[])
    return cfg, transformers.Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).eval()


@pytest.mark.parametrize("sharded", [True, False])
def test_load_skeleton_qwen3_takes_every_non_expert_tensor(tmp_path, sharded):
    cfg, model = tiny_qwen3()
    write_checkpoint(tmp_path, cfg, qwen3_checkpoint_tensors(model), sharded)
    ck = SafetensorsDir(str(tmp_path))
    assert ("model.layers.0.mlp.experts.3.down_proj.weight" in ck) and len(ck.names()) > 20
    rt = Runtime(None)
    got, gcfg = load_skeleton(str(tmp_path), rt, device="cpu")
    assert gcfg.num_experts == 4 and all(isinstance(lay.mlp, PagedMoEBlock) for lay in got.model.layers)
    assert all(lay.mlp.rt is rt for lay in got.model.layers)
    ref = {k: v for k, v in model.state_dict().items() if ".mlp.experts." not in k}
    have = got.state_dict()
    assert set(ref) == set(have)
    for k, v in ref.items():
        assert have[k].dtype == torch.bfloat16 and torch.equal(have[k], v), k
    assert not any(p.is_meta for p in got.parameters())
    assert got.model.rotary_emb.inv_freq.dtype == torch.float32


def test_load_skeleton_names_a_missing_tensor(tmp_path):
    cfg, model = tiny_qwen3()
    tensors = qwen3_checkpoint_tensors(model)
    del tensors["model.layers.1.self_attn.o_proj.weight"]
    write_checkpoint(tmp_path, cfg, tensors, sharded=False)
    with pytest.raises(KeyError, match="o_proj"):
        load_skeleton(str(tmp_path), Runtime(None), device="cpu")


def test_load_skeleton_gptoss_takes_non_experts_and_biases(tmp_path):
    torch.manual_seed(1)
    cfg = transformers.GptOssConfig(vocab_size=96, hidden_size=64, intermediate_size=64, num_hidden_layers=2,
                                    num_attention_heads=4, num_key_value_heads=2, head_dim=16, num_local_experts=4,
                                    num_experts_per_tok=2, max_position_embeddings=128,
                                    layer_types=["sliding_attention", "full_attention"])
    model = transformers.GptOssForCausalLM(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():
        for p in model.parameters():  # transformers leaves some at zero; every tensor distinct here
            p.copy_(torch.randn_like(p.float()).to(p.dtype))
    write_checkpoint(tmp_path, cfg, model.state_dict(), sharded=True)
    got, _ = load_skeleton(str(tmp_path), Runtime(None), device="cpu")  # dispatches on model_type
    assert all(isinstance(lay.mlp, PagedGptOssBlock) for lay in got.model.layers)
    ref = model.state_dict()
    have = got.state_dict()
    for k, v in ref.items():
        if ".mlp.experts." in k:
            continue
        assert torch.equal(have[k], v), k
    for l, lay in enumerate(got.model.layers):
        p = f"model.layers.{l}.mlp.experts."
        assert torch.equal(lay.mlp.gub, ref[p + "gate_up_proj_bias"])
        assert torch.equal(lay.mlp.db, ref[p + "down_proj_bias"])
