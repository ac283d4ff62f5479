"""gpt-oss adapter (openai/gpt-oss-20b and -120b) on the WiSP expert store, cache and
slot pool. Same interface as the reference's wisp/gptoss.py (gptoss.py:1-183).

An expert is gate_up [H, 2I] (gate and up interleaved on the last axis), down [I, H],
plus two biases. With I == H both halves of gate_up and down are n = H*I elements, so
an expert fits the flat [3, n] layout [gate_up.flat[:n] | gate_up.flat[n:] | down.flat]
(gptoss.py:32-37) and the store, cache and quantizer are reused unchanged; the biases
stay on the GPU for all experts.

Execution of PagedGptOssBlock.forward (all on the GPU; there is no CPU path):
  * one token, 4/3/2-bit experts: the three gfx950 decode kernels of
    kernels.gptoss_decode on the slot pool (bf16 weights dequantized in registers, the
    reference's bf16 rounding of every intermediate, one host sync per layer);
  * otherwise (several tokens, 16/8-bit stores, decode-on-load): the reference's
    dequantize-then-matmul path (bit-exact dequant kernel + bf16 GEMMs).
MXFP4 checkpoint tensors are decoded by a HIP kernel (kernels.mxfp4_to_bf16).
"""

from __future__ import annotations

import json
import os
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

from .store import ExpertStore

# e2m1 code -> value (gptoss.py:19)
FP4 = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def mxfp4_to_bf16(blocks, scales):
    """gptoss.py:22-29: blocks [..., G, 16] uint8 (two fp4 per byte, low nibble first),
    scales [..., G] uint8 (power-of-two exponents, bias 127) -> [..., G*32] bfloat16."""
    from .kernels import mxfp4_to_bf16 as _k

    return _k(blocks, scales)


def expert_w3(gate_up, down):
    """gate_up [H, 2I], down [I, H] -> [3, n] (n = H*I), gptoss.py:32-37."""
    H, I2 = gate_up.shape
    n = H * (I2 // 2)
    f = gate_up.reshape(-1)
    return torch.stack([f[:n], f[n:], down.reshape(-1)])


def _layer_tensors(get, has, l, E, device):
    """Dequantized gate_up [E, H, 2I], down [E, I, H], biases, for one layer (MXFP4 or
    plain bf16 checkpoints), gptoss.py:40-49."""
    p = f"model.layers.{l}.mlp.experts."
    if has(p + "gate_up_proj_blocks"):
        gu = mxfp4_to_bf16(get(p + "gate_up_proj_blocks").to(device), get(p + "gate_up_proj_scales").to(device))
        dn = mxfp4_to_bf16(get(p + "down_proj_blocks").to(device), get(p + "down_proj_scales").to(device))
        gu, dn = gu.transpose(1, 2).contiguous(), dn.transpose(1, 2).contiguous()  # [E,out,K] -> [E,K,out]
    else:
        gu, dn = get(p + "gate_up_proj").to(device), get(p + "down_proj").to(device)
    return gu, dn, get(p + "gate_up_proj_bias"), get(p + "down_proj_bias")


def _reader(model_dir):
    """Tensor getter over model.safetensors.index.json (gptoss.py:52-63)."""
    from safetensors import safe_open

    with open(os.path.join(model_dir, "model.safetensors.index.json")) as f:
        idx = json.load(f)["weight_map"]
    handles = {}

    def get(name):
        fn = idx[name]
        if fn not in handles:
            handles[fn] = safe_open(os.path.join(model_dir, fn), framework="pt", device="cpu")
        return handles[fn].get_tensor(name)

    return get, (lambda name: name in idx), idx


def build_store(model_dir, cfg, bits, group=128, device="cuda", cache_dir=None, pin=True):
    """All experts of a gpt-oss checkpoint, quantized on the GPU into an ExpertStore, cached
    on disk as raw rows under cache_dir (gptoss.py:66-89)."""
    L, E, H, I = cfg.num_hidden_layers, cfg.num_local_experts, cfg.hidden_size, cfg.intermediate_size
    if H != I:
        raise ValueError("the gpt-oss adapter needs intermediate_size == hidden_size (true for gpt-oss)")
    n = H * I
    st = ExpertStore(L, E, n, bits, group, pin)
    path = None
    if cache_dir and bits < 16:
        os.makedirs(cache_dir, exist_ok=True)
        path = os.path.join(cache_dir, f"store_gptoss_b{bits}_g{group}_{L}x{E}x{n}.u8")
        if os.path.exists(path) and os.path.getsize(path) == st.host.numel():
            st._load(path)
            return st
    get, has, _ = _reader(model_dir)
    t0 = time.time()
    for l in range(L):
        gu, dn, _, _ = _layer_tensors(get, has, l, E, device)
        for e in range(E):
            st.put(l, e, expert_w3(gu[e], dn[e]), device)
        del gu, dn
        if l % 4 == 3 or l == L - 1:
            print(f"[store] gpt-oss bits={bits} layer {l + 1}/{L}  {time.time() - t0:.0f}s", flush=True)
    if path:
        st._save(path)
    return st


class PagedGptOssBlock(nn.Module):
    """Drop-in for GptOssMLP: the router stays resident, the experts are paged
    (gptoss.py:92-143). Returns (output, router_scores) like transformers."""

    def __init__(self, router, layer_idx, rt, cfg, device="cuda"):
        super().__init__()
        self.router, self.layer_idx, self.rt = router, layer_idx, rt
        self.E, self.top_k = cfg.num_local_experts, cfg.num_experts_per_tok
        self.H, self.I = cfg.hidden_size, cfg.intermediate_size
        self.alpha, self.limit = 1.702, float(getattr(cfg, "swiglu_limit", 7.0))
        self.register_buffer(
            "gub", torch.zeros(self.E, 2 * self.I, dtype=torch.bfloat16, device=device), persistent=False
        )
        self.register_buffer("db", torch.zeros(self.E, self.H, dtype=torch.bfloat16, device=device), persistent=False)

    def _act(self, gu):
        """Clamped SwiGLU on interleaved gate/up (gptoss.py:120-122)."""
        gate, up = gu[..., ::2].clamp(max=self.limit), gu[..., 1::2].clamp(min=-self.limit, max=self.limit)
        return (up + 1) * (gate * torch.sigmoid(gate * self.alpha))

    def _fused_ok(self, cache):
        st = cache.store
        return (st.bits in (2, 3, 4) and not cache.decode_on_load and self.H % 32 == 0 and self.I % 16 == 0
                and st.group % 32 == 0)

    def forward(self, hidden_states):
        rt, cache = self.rt, self.rt.cache
        B, T, H = hidden_states.shape
        x = hidden_states.reshape(-1, H)
        N, k, I = x.shape[0], self.top_k, self.I
        logits = F.linear(x, self.router.weight, self.router.bias)
        tv, ti = torch.topk(logits, k, dim=-1)
        sc = F.softmax(tv, dim=1, dtype=tv.dtype)
        base = self.layer_idx * self.E
        rt.stats["layer_calls"] += 1
        if N == 1 and self._fused_ok(cache):
            row = torch.cat([ti.float(), sc.float()], 1).cpu()[0]  # the single sync of this layer
            ex = row[:k].to(torch.int64)
            if rt.recorder is not None:
                rt.recorder.append((self.layer_idx, ex.view(1, k).numpy().copy()))
            slots = cache.ensure([base + int(e) for e in ex])
            meta = torch.cat([torch.tensor(slots, dtype=torch.float32), row[k:], row[:k]]).pin_memory()
            meta = meta.to(x.device, non_blocking=True)
            from .kernels import gptoss_decode

            st = cache.store
            y = gptoss_decode(cache.gpu, meta, x[0], self.gub, self.db, k, st.n, H, I, st.bits, st.group,
                              self.alpha, self.limit).view(1, H)
            rt.stats["gpu_experts"] += k
        elif N == 1:  # decode through the reference's dequantize + 2 bmm path
            if rt.recorder is not None:
                rt.recorder.append((self.layer_idx, ti.cpu().numpy().copy()))
            ex = ti[0].tolist()
            slots = cache.ensure([base + e for e in ex])
            W = cache.weights_batched(torch.as_tensor(slots, device=x.device))  # [k, 3, n]
            # contiguous operands: bf16 batched products on strided views are avoided on this platform
            xk = x.unsqueeze(0).expand(k, 1, H).contiguous()
            gu = torch.bmm(xk, W[:, :2].reshape(k, H, 2 * I).contiguous()) + self.gub[ti[0]].unsqueeze(1)
            out = torch.bmm(self._act(gu).contiguous(), W[:, 2].reshape(k, I, H).contiguous()) + self.db[ti[0]].unsqueeze(1)
            y = (out[:, 0] * sc[0].unsqueeze(-1)).sum(0, keepdim=True)
            rt.stats["gpu_experts"] += k
        else:  # prefill: group tokens per expert, page in chunks
            if rt.recorder is not None:
                rt.recorder.append((self.layer_idx, ti.cpu().numpy().copy()))
            y = torch.zeros_like(x)
            uniq = torch.unique(ti).tolist()
            for i in range(0, len(uniq), rt.chunk):
                ce = uniq[i : i + rt.chunk]
                Ws = cache.weights(cache.ensure([base + e for e in ce]))
                for e, W3 in zip(ce, Ws, strict=True):
                    tok, pos = torch.where(ti == e)
                    gu = x[tok] @ torch.cat([W3[0], W3[1]]).view(H, 2 * I) + self.gub[e]
                    out = self._act(gu) @ W3[2].view(I, H) + self.db[e]
                    y.index_add_(0, tok, (out * sc[tok, pos, None]).to(x.dtype))
                    rt.stats["gpu_experts"] += 1
        return y.view(B, T, H), sc


def load_skeleton_gptoss(model_dir, rt, device="cuda"):
    """Meta-init the transformers gpt-oss model, swap every MLP for a paged block, load all
    non-expert tensors and the expert biases (gptoss.py:146-183)."""
    from transformers import AutoConfig, AutoModelForCausalLM
    from safetensors import safe_open

    from .model import nbytes_of

    cfg = AutoConfig.from_pretrained(model_dir)
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.bfloat16)
    blocks = []
    for i, layer in enumerate(model.model.layers):
        blk = PagedGptOssBlock(layer.mlp.router, i, rt, cfg, device)
        layer.mlp = blk
        blocks.append(blk)
    get, has, idx = _reader(model_dir)
    wanted = {k: f for k, f in idx.items() if ".mlp.experts." not in k}
    sd, t0 = {}, time.time()
    for fn in sorted(set(wanted.values())):
        with safe_open(os.path.join(model_dir, fn), framework="pt", device=str(device)) as h:
            for key in h.keys():
                if key in wanted:
                    sd[key] = h.get_tensor(key)
    res = model.load_state_dict(sd, strict=False, assign=True)
    bad = [key for key in res.missing_keys if "rotary" not in key]
    if bad:
        raise RuntimeError(f"missing keys: {bad[:5]}")
    for l, blk in enumerate(blocks):
        p = f"model.layers.{l}.mlp.experts."
        blk.gub.copy_(get(p + "gate_up_proj_bias").to(device))
        blk.db.copy_(get(p + "down_proj_bias").to(device))
    model.model.rotary_emb = type(model.model.rotary_emb)(config=cfg, device=device)
    model.eval()
    print(f"[model] gpt-oss non-expert weights on {device}: {nbytes_of(model) / 2**30:.2f} GiB "
          f"({time.time() - t0:.0f}s)", flush=True)
    return model, cfg
