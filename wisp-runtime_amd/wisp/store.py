"""The quantized experts of every layer, in pinned host memory: the source the expert cache
pages from. Reference interface: wisp/store.py:12-110 (ExpertStore: L, E, n, bits, group,
nbytes, host, pinned, total_gib, key, put, from_experts, from_safetensors, _save, _load);
same row format.

Layout. One row of `nbytes = expert_nbytes(n, bits, group)` bytes per (layer, expert) at
row `key = layer * E + expert`, all rows in ONE page-locked allocation, so a cache miss is
a single contiguous read of `nbytes` at `key * nbytes` -- by a DMA copy or by the GPU's
page kernel reading the pinned rows directly over PCIe.

Filling. `fill` quantizes experts on the GPU with the package's bit-exact kernel into a
ring of device staging rows and copies each finished row to its pinned row on a side
stream, so the PCIe transfer of one expert overlaps the quantization of the next ones;
the host never waits per expert.

Checkpoints. `from_safetensors` quantizes the experts of a Qwen3-MoE safetensors checkpoint
through `fill` (per-expert tensors as published, or per-layer fused ones as newer
transformers write them); `SafetensorsDir` reads a checkpoint directory by tensor name.

Persistence. A `.u8` file is the rows back to back with no header (its size identifies the
shape: L * E * nbytes). `save` writes through a temporary file renamed into place; both
directions stream 64 MiB at a time, so a 15 GB store never needs a second copy in memory.
"""

from __future__ import annotations

import json
import os
import time
from typing import Iterable

import torch

from .quant import expert_nbytes, quantize

_IO_PIECE = 64 << 20  # bytes per read/write call of save/load


def _host_rows(nrows: int, nbytes: int, pin: bool):
    """[nrows, nbytes] uint8 on the host, page-locked when `pin` and the runtime allows it.
    Returns (tensor, pinned). A pageable store still works with DMA copies; the page
    kernel (ExpertCache copy="kernel") needs a pinned one."""
    if pin:
        try:
            return torch.empty((nrows, nbytes), dtype=torch.uint8, pin_memory=True), True
        except RuntimeError as err:
            print(f"[store] page-locked allocation refused ({err}); the store is pageable", flush=True)
    return torch.empty((nrows, nbytes), dtype=torch.uint8), False


class SafetensorsDir:
    """The tensors of a safetensors checkpoint directory by name: the weight map of
    model.safetensors.index.json (a sharded checkpoint) or the names in the one
    model.safetensors. Each file is opened once; `get` reads one tensor to the CPU,
    `load` many straight to a device (the reference's _reader, gptoss.py:52-64, and the
    loops of model.py:37-43)."""

    def __init__(self, model_dir):
        from safetensors import safe_open

        self.dir, self._open = model_dir, {}
        index = os.path.join(model_dir, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                self.files = dict(json.load(f)["weight_map"])
        else:
            with safe_open(os.path.join(model_dir, "model.safetensors"), framework="pt") as h:
                self.files = {name: "model.safetensors" for name in h.keys()}

    def __contains__(self, name) -> bool:
        return name in self.files

    def names(self):
        return list(self.files)

    def get(self, name) -> torch.Tensor:
        from safetensors import safe_open

        f = self.files[name]
        h = self._open.get(f)
        if h is None:
            h = self._open[f] = safe_open(os.path.join(self.dir, f), framework="pt", device="cpu")
        return h.get_tensor(name)

    def load(self, names, device="cpu") -> dict:
        """{name: tensor on `device`} for `names`, one pass over each file that holds some."""
        from safetensors import safe_open

        by_file = {}
        for name in names:
            by_file.setdefault(self.files[name], []).append(name)
        out = {}
        for f, group in sorted(by_file.items()):
            with safe_open(os.path.join(self.dir, f), framework="pt", device=str(device)) as h:
                for name in group:
                    out[name] = h.get_tensor(name)
        return out


class ExpertStore:
    def __init__(self, n_layers, n_experts, n, bits, group=128, pin=True):
        self.L, self.E, self.n, self.bits, self.group = n_layers, n_experts, n, bits, group
        self.nbytes = expert_nbytes(n, bits, group)
        t0 = time.time()
        self.host, self.pinned = _host_rows(n_layers * n_experts, self.nbytes, pin)
        print(f"[store] {n_layers}x{n_experts} experts, {self.total_gib:.1f} GiB host (pinned={self.pinned}) "
              f"in {time.time() - t0:.1f}s", flush=True)

    @property
    def total_gib(self) -> float:
        return self.host.numel() / 2**30

    @property
    def rows(self) -> int:
        return self.host.shape[0]

    def key(self, l: int, e: int) -> int:
        """Row of expert e of layer l (the key the cache and the graph decoder use)."""
        return l * self.E + e

    # ---------------------------------------------------------------- filling
    @torch.no_grad()
    def fill(self, items: Iterable, device="cuda", ring: int = 4) -> int:
        """Quantize experts into their rows. items: iterable of (key, w3) with w3 [3, n] of any
        float dtype (on any device; moved to `device`). Up to `ring` rows are in flight: row i
        is quantized into staging slot i % ring on the current stream, then copied to the pinned
        row on a side stream that waits only for that quantization. Returns the row count."""
        side = None
        count = 0
        for key, w3 in items:
            if not 0 <= key < self.rows:
                raise IndexError(f"expert row {key} outside the store's {self.rows} rows")
            if side is None:  # device state on the first row (the quantizer has no CPU path)
                dev = torch.device(device)
                if dev.type != "cuda":
                    raise RuntimeError("ExpertStore.fill quantizes on a ROCm device; no CPU path is provided")
                if dev.index is None:
                    dev = torch.device("cuda", torch.cuda.current_device())
                compute = torch.cuda.current_stream(dev)
                side = torch.cuda.Stream(dev)
                staging = torch.empty((ring, self.nbytes), dtype=torch.uint8, device=dev)
                free = [torch.cuda.Event() for _ in range(ring)]  # copy of slot s done: it may be rewritten
                used = [False] * ring
            s = count % ring
            if used[s]:
                compute.wait_event(free[s])
            quantize(w3.to(dev), self.bits, self.group, out=staging[s])
            done = torch.cuda.Event()
            done.record(compute)
            side.wait_event(done)
            with torch.cuda.stream(side):
                self.host[key].copy_(staging[s], non_blocking=self.pinned)
                free[s].record(side)
            used[s] = True
            count += 1
        if side is not None:
            side.synchronize()
        return count

    def put(self, l, e, w3, device="cuda"):
        """Quantize expert (l, e) from w3 [3, n] on `device` into its row."""
        self.fill([(self.key(l, e), w3)], device, ring=1)

    @classmethod
    def from_experts(cls, layers, bits, group=128, device="cuda", pin=True):
        """layers: per layer, a list of (gate_w, up_w, down_w) weight tensors of one shape."""
        n = layers[0][0][0].numel()
        st = cls(len(layers), len(layers[0]), n, bits, group, pin)
        st.fill(((st.key(l, e), torch.stack([g.reshape(-1), u.reshape(-1), d.reshape(-1)]))
                 for l, exps in enumerate(layers) for e, (g, u, d) in enumerate(exps)), device)
        return st

    @classmethod
    def from_safetensors(cls, model_dir, cfg, bits, group=128, device="cuda", cache_dir=None, pin=True):
        """The experts of a Qwen3-MoE checkpoint quantized into a new store (store.py:54-93).
        Expert tensors per expert (model.layers.{l}.mlp.experts.{e}.gate_proj / up_proj /
        down_proj .weight, as published) or fused per layer (experts.gate_up_proj [E, 2I, H],
        gate rows first, and experts.down_proj [E, H, I]). With cache_dir (and bits < 16) the
        rows are read from, or else written to, the reference's cache file of this shape."""
        L, E = cfg.num_hidden_layers, cfg.num_experts
        H, I = cfg.hidden_size, cfg.moe_intermediate_size
        st = cls(L, E, H * I, bits, group, pin)
        path = None
        if cache_dir and bits < 16:
            os.makedirs(cache_dir, exist_ok=True)
            path = cls.cache_file(cache_dir, bits, group, L, E, H * I)
            if os.path.exists(path) and os.path.getsize(path) == st.host.numel():
                st.load(path)
                return st
        ck = SafetensorsDir(model_dir)

        def experts():
            for l in range(L):
                p = f"model.layers.{l}.mlp.experts."
                if p + "gate_up_proj" in ck:
                    gu, dn = ck.get(p + "gate_up_proj"), ck.get(p + "down_proj")
                    assert gu.shape == (E, 2 * I, H) and dn.shape == (E, H, I), (gu.shape, dn.shape)
                    for e in range(E):
                        yield st.key(l, e), torch.stack([gu[e, :I].reshape(-1), gu[e, I:].reshape(-1),
                                                         dn[e].reshape(-1)])
                else:
                    for e in range(E):
                        q = f"{p}{e}."
                        yield st.key(l, e), torch.stack([ck.get(q + "gate_proj.weight").reshape(-1),
                                                         ck.get(q + "up_proj.weight").reshape(-1),
                                                         ck.get(q + "down_proj.weight").reshape(-1)])

        st.fill(experts(), device)
        if path:
            st.save(path)
        return st

    # ---------------------------------------------------------------- persistence
    @staticmethod
    def cache_file(cache_dir: str, bits: int, group: int, L: int, E: int, n: int) -> str:
        """Where a store of this shape is cached (the reference's file name, store.py:62)."""
        return os.path.join(cache_dir, f"store_b{bits}_g{group}_{L}x{E}x{n}.u8")

    def _flat(self) -> memoryview:
        return memoryview(self.host.numpy()).cast("B")

    def save(self, path: str) -> None:
        """Write the rows back to back (no header) to `path`, atomically (temp file + rename)."""
        buf = self._flat()
        tmp = path + ".tmp"
        with open(tmp, "wb") as f:
            for off in range(0, len(buf), _IO_PIECE):
                f.write(buf[off : off + _IO_PIECE])
        os.replace(tmp, path)

    def load(self, path: str) -> None:
        """Read a file written by `save` (or the reference's `_save`) into the rows. The file
        must hold exactly L * E * nbytes bytes."""
        size = os.path.getsize(path)
        if size != self.host.numel():
            raise ValueError(f"{path}: {size} bytes, this store holds {self.host.numel()} "
                             f"({self.rows} rows of {self.nbytes})")
        buf = self._flat()
        with open(path, "rb") as f:
            off = 0
            while off < len(buf):
                got = f.readinto(buf[off : off + _IO_PIECE])
                if not got:
                    raise IOError(f"{path}: short read at byte {off}")
                off += got

    # the reference's names (store.py:96-110)
    def _save(self, path, rows=None):
        self.save(path)

    def _load(self, path, rows=None):
        self.load(path)
