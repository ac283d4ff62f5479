"""gpt-oss experts (openai/gpt-oss-20b and -120b) on this package's expert store, cache and
slot pool. Reference interface: wisp/gptoss.py (mxfp4_to_bf16 :22-29, expert_w3 :32-37,
PagedGptOssBlock :92-143).

Expert format. A gpt-oss expert is gate_up [H, 2I] (gate and up interleaved along the last
axis), down [I, H], and bf16 biases gate_up [2I] and down [H]. gpt-oss has I == H, so each
half of gate_up and the down matrix hold n = H*I elements, and an expert is stored in the
flat [3, n] format every other expert of this package uses:
    [ gate_up.flat[:n] | gate_up.flat[n:] | down.flat ]
so the quantizer, store, cache and page kernel serve it unchanged. The biases of all
experts stay on the GPU in the block.

PagedGptOssBlock.forward:
  * routing: router logits (with bias), the k largest, softmax over those k in the
    activation dtype; the scores are returned beside the output, as transformers does;
  * one token with 2/3/4-bit experts in the pool: the three gfx950 decode launches of
    kernels.gptoss_decode (weights dequantized in registers, the reference's bf16
    rounding of every intermediate);
  * any other case (several tokens, 8/16-bit stores, decode-on-load): every routed
    (token, expert) pair exactly once, grouped per expert by one stable sort of the routing;
    experts are paged rt.chunk at a time and run as bf16 GEMMs on their bit-exactly
    dequantized weights.
Checkpoints: build_store quantizes the experts of a gpt-oss safetensors checkpoint (MXFP4
blocks and scales, decoded by the HIP kernel kernels.mxfp4_to_bf16, or plain bf16) into an
ExpertStore (gptoss.py:67-90), and load_skeleton_gptoss builds the model with paged blocks
and loads its non-expert tensors and the expert biases (gptoss.py:146-176).
"""

from __future__ import annotations

import os
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

# e2m1 code -> value (gptoss.py:19); the decode kernel holds the same table
FP4 = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def mxfp4_to_bf16(blocks, scales):
    """blocks [..., G, 16] uint8 (two e2m1 codes per byte, low nibble first), scales [..., G]
    uint8 (power-of-two exponents, bias 127) -> [..., G*32] bfloat16, on the GPU."""
    from .kernels import mxfp4_to_bf16 as decode

    return decode(blocks, scales)


def expert_w3(gate_up, down):
    """gate_up [H, 2I] and down [I, H] of one expert -> the flat [3, n] rows, n = H*I."""
    half = gate_up.numel() // 2
    flat = gate_up.reshape(-1)
    return torch.stack([flat[:half], flat[half:], down.reshape(-1)])


def _layer_experts(ck, l, device):
    """gate_up [E, H, 2I] and down [E, I, H] (bf16, on `device`) of layer l of checkpoint ck
    (a SafetensorsDir): MXFP4 blocks [E, out, K/32, 16] + scales [E, out, K/32] decoded and
    transposed to [E, K, out], or the plain tensors (gptoss.py:38-49)."""
    p = f"model.layers.{l}.mlp.experts."
    if p + "gate_up_proj_blocks" in ck:
        gu = mxfp4_to_bf16(ck.get(p + "gate_up_proj_blocks").to(device), ck.get(p + "gate_up_proj_scales").to(device))
        dn = mxfp4_to_bf16(ck.get(p + "down_proj_blocks").to(device), ck.get(p + "down_proj_scales").to(device))
        return gu.transpose(1, 2).contiguous(), dn.transpose(1, 2).contiguous()
    return ck.get(p + "gate_up_proj").to(device), ck.get(p + "down_proj").to(device)


def build_store(model_dir, cfg, bits, group=128, device="cuda", cache_dir=None, pin=True):
    """The experts of a gpt-oss checkpoint quantized into a new ExpertStore of [3, H*I] rows
    (gptoss.py:67-90; gpt-oss has I == H). With cache_dir (and bits < 16) the rows are read
    from, or else written to, a cache file of this shape."""
    from .store import ExpertStore, SafetensorsDir

    L, E, H, I = cfg.num_hidden_layers, cfg.num_local_experts, cfg.hidden_size, cfg.intermediate_size
    if H != I:
        raise ValueError(f"the [3, n] expert rows need intermediate_size == hidden_size (gpt-oss): {I} != {H}")
    st = ExpertStore(L, E, H * I, bits, group, pin)
    path = None
    if cache_dir and bits < 16:
        os.makedirs(cache_dir, exist_ok=True)
        path = os.path.join(cache_dir, f"store_gptoss_b{bits}_g{group}_{L}x{E}x{H * I}.u8")
        if os.path.exists(path) and os.path.getsize(path) == st.host.numel():
            st.load(path)
            return st
    ck = SafetensorsDir(model_dir)
    for l in range(L):
        gu, dn = _layer_experts(ck, l, device)
        st.fill(((st.key(l, e), expert_w3(gu[e], dn[e])) for e in range(E)), device)
        del gu, dn
    if path:
        st.save(path)
    return st


@torch.no_grad()
def load_skeleton_gptoss(model_dir, rt, device="cuda"):
    """gpt-oss built on the meta device with every MLP replaced by a PagedGptOssBlock on rt,
    the non-expert tensors and the experts' biases loaded to `device` (gptoss.py:146-176).
    Returns (model, cfg)."""
    from transformers import AutoConfig, AutoModelForCausalLM

    from .model import _fresh_rotary, _load_non_experts, nbytes_of
    from .store import SafetensorsDir

    cfg = AutoConfig.from_pretrained(model_dir)
    t0 = time.time()
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16)
    blocks = []
    for i, layer in enumerate(model.model.layers):
        layer.mlp = PagedGptOssBlock(layer.mlp.router, i, rt, cfg, device)
        blocks.append(layer.mlp)
    ck = SafetensorsDir(model_dir)
    _load_non_experts(model, ck, device)
    for l, blk in enumerate(blocks):
        p = f"model.layers.{l}.mlp.experts."
        blk.gub.copy_(ck.get(p + "gate_up_proj_bias"))
        blk.db.copy_(ck.get(p + "down_proj_bias"))
    _fresh_rotary(model, cfg, device)
    model.eval()
    print(f"[model] gpt-oss non-expert weights on {device}: {nbytes_of(model) / 2**30:.2f} GiB "
          f"({time.time() - t0:.0f}s)", flush=True)
    return model, cfg


def clamped_swiglu(gu, alpha: float, limit: float):
    """gpt-oss's activation on interleaved gate/up columns (gptoss.py:120-122): gate clamped
    from above at `limit`, up clamped to [-limit, limit], (up + 1) * gate * sigmoid(alpha*gate)."""
    gate = torch.clamp(gu[..., 0::2], max=limit)
    up = torch.clamp(gu[..., 1::2], -limit, limit)
    return (up + 1) * (gate * torch.sigmoid(gate * alpha))


class PagedGptOssBlock(nn.Module):
    """Drop-in for transformers' GptOssMLP: the router stays resident, the experts are paged
    from the store. Returns (output [B, T, H], router scores [B*T, k])."""

    def __init__(self, router, layer_idx, rt, cfg, device="cuda"):
        super().__init__()
        self.router, self.layer_idx, self.rt = router, layer_idx, rt
        self.E, self.top_k = cfg.num_local_experts, cfg.num_experts_per_tok
        self.H, self.I = cfg.hidden_size, cfg.intermediate_size
        self.alpha, self.limit = 1.702, float(getattr(cfg, "swiglu_limit", 7.0))
        bf = dict(dtype=torch.bfloat16, device=device)
        self.register_buffer("gub", torch.zeros(self.E, 2 * self.I, **bf), persistent=False)
        self.register_buffer("db", torch.zeros(self.E, self.H, **bf), persistent=False)

    def _act(self, gu):
        return clamped_swiglu(gu, self.alpha, self.limit)

    def _fused_ok(self, cache):
        """Whether one token can take the fused decode kernels on this cache's pool."""
        st = cache.store
        return (st.bits in (2, 3, 4) and not cache.decode_on_load and self.H % 32 == 0 and self.I % 16 == 0
                and st.group % 32 == 0)

    def forward(self, hidden_states):
        rt, cache = self.rt, self.rt.cache
        B, T, H = hidden_states.shape
        x = hidden_states.reshape(-1, H)
        k = self.top_k
        top_logits, ids = torch.topk(F.linear(x, self.router.weight, self.router.bias), k, dim=-1)
        scores = F.softmax(top_logits, dim=1, dtype=top_logits.dtype)
        rt.stats["layer_calls"] += 1
        if x.shape[0] == 1 and self._fused_ok(cache):
            y = self._decode_fused(x, ids, scores)
        else:
            y = self._grouped(x, ids, scores)
        return y.view(B, T, H), scores

    def _record(self, ids_cpu):
        if self.rt.recorder is not None:
            self.rt.recorder.append((self.layer_idx, ids_cpu.numpy().copy()))

    def _decode_fused(self, x, ids, scores):
        """One token: page the k experts, then the three decode launches read them in place."""
        rt, cache, k = self.rt, self.rt.cache, self.top_k
        row = torch.cat([ids.float(), scores.float()], 1).cpu()[0]  # the layer's one host sync
        ex = row[:k].to(torch.int64)
        self._record(ex.view(1, k))
        slots = cache.ensure([self.layer_idx * self.E + int(e) for e in ex])
        # meta [slot ids | routing weights | expert ids] (the kernels index the biases by id)
        meta = torch.cat([torch.tensor(slots, dtype=torch.float32), row[k:], row[:k]]).pin_memory()
        meta = meta.to(x.device, non_blocking=True)
        from .kernels import gptoss_decode

        st = cache.store
        y = gptoss_decode(cache.gpu, meta, x[0], self.gub, self.db, k, st.n, self.H, self.I, st.bits, st.group,
                          self.alpha, self.limit)
        rt.stats["gpu_experts"] += k
        return y.view(1, self.H)

    def _grouped(self, x, ids, scores):
        """Every (token, expert) pair once: pairs sorted by expert (stable, so tokens stay in
        order within an expert), experts paged rt.chunk at a time and dequantized bit-exactly,
        then per expert gate_up GEMM + bias, activation, down GEMM + bias, and the weighted rows
        added to their tokens (the reference's bf16 rounding points, gptoss.py:131-143)."""
        rt, cache, k, H, I = self.rt, self.rt.cache, self.top_k, self.H, self.I
        N = x.shape[0]
        flat = ids.reshape(-1)
        order = torch.argsort(flat, stable=True)
        experts, counts = torch.unique_consecutive(flat[order], return_counts=True)
        experts, counts = experts.tolist(), counts.tolist()  # the layer's one host sync
        self._record(ids.cpu())
        tok_of_pair = order // k
        w_of_pair = scores.reshape(-1)[order]
        y = torch.zeros_like(x)
        starts = [0]
        for c in counts:
            starts.append(starts[-1] + c)
        base = self.layer_idx * self.E
        for c0 in range(0, len(experts), max(1, rt.chunk)):
            batch = experts[c0 : c0 + max(1, rt.chunk)]
            W = cache.weights(cache.ensure([base + e for e in batch]))
            for j, e in enumerate(batch):
                lo, hi = starts[c0 + j], starts[c0 + j + 1]
                tok = tok_of_pair[lo:hi]
                w_gu = W[j][:2].reshape(H, 2 * I)  # contiguous rows of the [3, n] expert
                w_dn = W[j][2].reshape(I, H)
                gu = x.index_select(0, tok) @ w_gu + self.gub[e]
                out = self._act(gu) @ w_dn + self.db[e]
                y.index_add_(0, tok, (out * w_of_pair[lo:hi, None]).to(x.dtype))
                rt.stats["gpu_experts"] += 1
        return y
