"""Expert stores built from safetensors checkpoints on the GPU: ExpertStore.from_safetensors
(the reference's store.py:54-93) on Qwen3-MoE experts named per expert and fused per layer,
and gptoss.build_store (gptoss.py:67-90) on MXFP4 blocks and on plain bf16 experts. Each
store's rows must equal, byte for byte, a store filled with the same expert weights through
`put`; the MXFP4 weights are decoded for that by the oracle (oracle.mxfp4_to_bf16_bits)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from test_checkpoint import qwen3_checkpoint_tensors, tiny_qwen3, write_checkpoint
from wisp.gptoss import build_store, expert_w3
from wisp.store import ExpertStore

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _rows_equal(a, b):
    return a.host.shape == b.host.shape and torch.equal(a.host, b.host)


@pytest.mark.parametrize("per_expert", [True, False])
@pytest.mark.parametrize("bits", [4, 3])
def test_from_safetensors_equals_put(tmp_path, per_expert, bits):
    cfg, model = tiny_qwen3(seed=bits)
    write_checkpoint(tmp_path / "ck", cfg, qwen3_checkpoint_tensors(model, per_expert), sharded=True)
    st = ExpertStore.from_safetensors(str(tmp_path / "ck"), cfg, bits, 128, cache_dir=str(tmp_path / "cache"))
    I = cfg.moe_intermediate_size
    ref = ExpertStore(cfg.num_hidden_layers, cfg.num_experts, cfg.hidden_size * I, bits, 128)
    for l, lay in enumerate(model.model.layers):
        ex = lay.mlp.experts
        for e in range(cfg.num_experts):
            ref.put(l, e, torch.stack([ex.gate_up_proj[e, :I].reshape(-1), ex.gate_up_proj[e, I:].reshape(-1),
                                       ex.down_proj[e].reshape(-1)]))
    assert _rows_equal(st, ref)
    again = ExpertStore.from_safetensors(str(tmp_path / "missing"), cfg, bits, 128, cache_dir=str(tmp_path / "cache"))
    assert _rows_equal(again, ref)  # read from the cache file: the checkpoint is not opened


def _gptoss_cfg(H=128, E=4, L=2):
    return transformers.GptOssConfig(vocab_size=64, hidden_size=H, intermediate_size=H, num_hidden_layers=L,
                                     num_attention_heads=4, num_key_value_heads=2, head_dim=32, num_local_experts=E,
                                     num_experts_per_tok=2, layer_types=["full_attention"] * L)


@pytest.mark.parametrize("mxfp4", [True, False])
def test_gptoss_build_store_equals_put(tmp_path, mxfp4):
    H, E, L = 128, 4, 2
    cfg = _gptoss_cfg(H, E, L)
    rng = np.random.default_rng(3)
    tensors, experts = {}, []
    for l in range(L):
        p = f"model.layers.{l}.mlp.experts."
        if mxfp4:  # [E, out, K/32, 16] codes and [E, out, K/32] exponents near 2^0
            gb = rng.integers(0, 256, (E, 2 * H, H // 32, 16), dtype=np.uint8)
            gs = rng.integers(118, 128, (E, 2 * H, H // 32), dtype=np.uint8)
            db = rng.integers(0, 256, (E, H, H // 32, 16), dtype=np.uint8)
            ds = rng.integers(118, 128, (E, H, H // 32), dtype=np.uint8)
            tensors.update({p + "gate_up_proj_blocks": torch.from_numpy(gb), p + "gate_up_proj_scales":
                            torch.from_numpy(gs), p + "down_proj_blocks": torch.from_numpy(db),
                            p + "down_proj_scales": torch.from_numpy(ds)})
            gu = torch.from_numpy(O.mxfp4_to_bf16_bits(gb, gs).view(np.int16)).view(torch.bfloat16).transpose(1, 2)
            dn = torch.from_numpy(O.mxfp4_to_bf16_bits(db, ds).view(np.int16)).view(torch.bfloat16).transpose(1, 2)
        else:
            gu = (torch.randn(E, H, 2 * H) * 0.05).to(torch.bfloat16)
            dn = (torch.randn(E, H, H) * 0.05).to(torch.bfloat16)
            tensors.update({p + "gate_up_proj": gu, p + "down_proj": dn})
        tensors[p + "gate_up_proj_bias"] = torch.zeros(E, 2 * H, dtype=torch.bfloat16)
        tensors[p + "down_proj_bias"] = torch.zeros(E, H, dtype=torch.bfloat16)
        experts.append((gu.contiguous(), dn.contiguous()))
    write_checkpoint(tmp_path / "ck", cfg, tensors, sharded=False)
    st = build_store(str(tmp_path / "ck"), cfg, 4, 128)
    ref = ExpertStore(L, E, H * H, 4, 128)
    for l, (gu, dn) in enumerate(experts):
        for e in range(E):
            ref.put(l, e, expert_w3(gu[e], dn[e]))
    assert _rows_equal(st, ref)
