"""Host-side store of all experts, quantized to `bits`, in pinned RAM.

Same interface as the reference's wisp/store.py (store.py:12-110): one row of
expert_nbytes per (layer, expert), key = layer * n_experts + expert, built by
quantizing on the GPU (this package's bit-exact kernels) and copying to the host,
cached on disk as raw rows (`.u8`, row after row, no header).
"""

from __future__ import annotations

import json
import os
import time

import torch

from .quant import expert_nbytes, quantize


class ExpertStore:
    def __init__(self, n_layers, n_experts, n, bits, group=128, pin=True):
        self.L, self.E, self.n, self.bits, self.group = n_layers, n_experts, n, bits, group
        self.nbytes = expert_nbytes(n, bits, group)
        t = time.time()
        try:
            self.host = torch.empty((n_layers * n_experts, self.nbytes), dtype=torch.uint8, pin_memory=pin)
            self.pinned = pin
        except RuntimeError as e:  # pinning refused: pageable rows still work, copies are slower
            print(f"[store] pin_memory failed ({e}); using pageable memory", flush=True)
            self.host = torch.empty((n_layers * n_experts, self.nbytes), dtype=torch.uint8)
            self.pinned = False
        print(f"[store] allocated {self.host.numel() / 2**30:.1f} GiB host (pinned={self.pinned}) "
              f"in {time.time() - t:.1f}s", flush=True)

    @property
    def total_gib(self):
        return self.host.numel() / 2**30

    def key(self, l, e):
        return l * self.E + e

    @torch.no_grad()
    def put(self, l, e, w3, device):
        """Quantize expert (l, e) from w3 [3, n] on `device` and store its row."""
        buf = quantize(w3.to(device), self.bits, self.group)
        self.host[self.key(l, e)].copy_(buf.cpu())

    # ---- builders -------------------------------------------------------
    @classmethod
    def from_experts(cls, layers, bits, group=128, device="cuda", pin=True):
        """layers: per layer, a list of (gate_w, up_w, down_w) tensors."""
        L, E = len(layers), len(layers[0])
        n = layers[0][0][0].numel()
        st = cls(L, E, n, bits, group, pin)
        for l, exps in enumerate(layers):
            for e, (g, u, d) in enumerate(exps):
                st.put(l, e, torch.stack([g.reshape(-1), u.reshape(-1), d.reshape(-1)]), device)
        return st

    @classmethod
    def from_safetensors(cls, model_dir, cfg, bits, group=128, device="cuda", cache_dir=None, pin=True):
        """Experts of a Qwen3-MoE checkpoint (`model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight`),
        read through model.safetensors.index.json; cached as raw rows under cache_dir."""
        from safetensors import safe_open

        L, E = cfg.num_hidden_layers, cfg.num_experts
        n = cfg.moe_intermediate_size * cfg.hidden_size
        st = cls(L, E, n, bits, group, pin)
        path = None
        if cache_dir and bits < 16:
            os.makedirs(cache_dir, exist_ok=True)
            path = os.path.join(cache_dir, f"store_b{bits}_g{group}_{L}x{E}x{n}.u8")
            if os.path.exists(path) and os.path.getsize(path) == st.host.numel():
                st._load(path)
                return st
        with open(os.path.join(model_dir, "model.safetensors.index.json")) as f:
            where = json.load(f)["weight_map"]
        files = {}

        def tensor(name):
            fn = where[name]
            if fn not in files:
                files[fn] = safe_open(os.path.join(model_dir, fn), framework="pt", device="cpu")
            return files[fn].get_tensor(name)

        t0 = time.time()
        for l in range(L):
            for e in range(E):
                p = f"model.layers.{l}.mlp.experts.{e}."
                w3 = torch.stack([tensor(p + m + "_proj.weight").reshape(-1) for m in ("gate", "up", "down")])
                st.put(l, e, w3, device)
            if l % 4 == 3 or l == L - 1:
                print(f"[store] bits={bits} layer {l + 1}/{L}  {time.time() - t0:.0f}s", flush=True)
        if path:
            st._save(path)
        return st

    # ---- persistence ----------------------------------------------------
    def _save(self, path, rows=256):
        a = self.host.numpy()
        with open(path + ".tmp", "wb") as f:
            for i in range(0, a.shape[0], rows):
                f.write(memoryview(a[i : i + rows]))
        os.replace(path + ".tmp", path)

    def _load(self, path, rows=256):
        a = self.host.numpy()
        with open(path, "rb") as f:
            for i in range(0, a.shape[0], rows):
                f.readinto(memoryview(a[i : i + rows]))
