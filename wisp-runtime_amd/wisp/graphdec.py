"""hipGraph decode of one token at batch 1, cut at the per-layer paging points.

Same interface as the reference's wisp/graphdec.py (GraphDecoder, graphdec.py:35-308).
A token needs one host decision per layer (which experts to page in), so the step is
split at those L points and everything between two of them is captured once as a
hipGraph and replayed:

    segment 0      embed -> attention(0) -> router(0)                       -> row
    (host)         row -> expert cache (native: ensure, copies, meta) -> meta_dev
    segment i      MoE(i-1) -> residual -> attention(i) -> router(i)        -> row
    segment L      MoE(L-1) -> residual -> final norm -> lm_head            -> logits

Every buffer a segment touches is static: the KV cache [1, Hk, Tmax, D] per layer, the
token and position in `ctl` (device), the routing in `meta_dev`. Attention always spans
the Tmax slots with the position read on the device, so the graphs do not depend on the
length. The decode segments run this package's gfx950 kernels: rope_decode,
attn_decode (grouped attention over the static cache), and the two MoE decode kernels
on the expert cache's slot pool. Prefill runs the model's own modules in chunks, with
attention computed in float32, writing K/V straight into the static buffers.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import kernels
from .moe import route


def _layer_kv(pk, i):
    """(keys, values) of layer i from a transformers cache object or a legacy tuple."""
    if hasattr(pk, "layers"):
        return pk.layers[i].keys, pk.layers[i].values
    if hasattr(pk, "key_cache"):
        return pk.key_cache[i], pk.value_cache[i]
    return pk[i][0], pk[i][1]


class GraphDecoder:
    def __init__(self, model, rt=None, tmax=2048, use_graph=True):
        cfg = model.config
        self.model, self.rt = model, rt
        self.L, self.H = cfg.num_hidden_layers, cfg.hidden_size
        self.Hq, self.Hk = cfg.num_attention_heads, cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or self.H // self.Hq
        self.G = self.Hq // self.Hk
        self.layers = list(model.model.layers)
        if not all(hasattr(l.mlp, "top_k") for l in self.layers):
            raise AssertionError("GraphDecoder needs an all-MoE model (paged MoE blocks in every layer)")
        blk = self.layers[0].mlp
        self.k = blk.top_k
        self.E = getattr(blk, "E", None) or cfg.num_experts
        emb = model.model.embed_tokens.weight
        self.dev, self.dt = emb.device, emb.dtype
        self.cuda = self.dev.type == "cuda"
        if not self.cuda:
            raise RuntimeError("GraphDecoder runs the gfx950 decode kernels: the model must be on a ROCm device")
        self.use_graph = use_graph
        self.kc = self.vc = None
        self.pos = 0
        self.ctl = torch.zeros(2, dtype=torch.long, device=self.dev)  # [token, position]
        self._alloc((tmax + 63) // 64 * 64)
        d = dict(device=self.dev, dtype=self.dt)
        self.hm = torch.zeros(1, 1, self.H, **d)  # residual stream after attention
        self.xn = torch.zeros(1, 1, self.H, **d)  # MoE input
        self.prefetch = bool(rt is not None and getattr(rt, "prefetch", False))
        self.row = torch.zeros(1, (3 if self.prefetch else 2) * self.k, dtype=torch.float32, device=self.dev)
        self.logits = torch.zeros(1, cfg.vocab_size, **d)
        self.meta_dev = torch.zeros(2 * self.k, dtype=torch.float32, device=self.dev)
        self.meta_host = torch.zeros(2 * self.k, dtype=torch.float32, pin_memory=True)
        self.graphs, self._key = None, None

    # ---------------------------------------------------------------- static buffers
    def _alloc(self, tmax):
        """(Re)allocate the static KV buffers for `tmax` positions, keeping the first `pos`."""
        d = dict(device=self.dev, dtype=self.dt)
        keep = min(self.pos, tmax)
        old_k, old_v = self.kc, self.vc
        self.kc, self.vc = [], []
        for i in range(self.L):
            kb = torch.zeros(1, self.Hk, tmax, self.D, **d)
            vb = torch.zeros(1, self.Hk, tmax, self.D, **d)
            if old_k is not None and keep:
                kb[:, :, :keep].copy_(old_k[i][:, :, :keep])
                vb[:, :, :keep].copy_(old_v[i][:, :, :keep])
                old_k[i] = old_v[i] = None  # release layer by layer
            self.kc.append(kb)
            self.vc.append(vb)
        self.tmax, self.pos = tmax, keep
        positions = torch.arange(tmax, device=self.dev)[None]
        cos, sin = self.model.model.rotary_emb(torch.zeros(1, 1, self.H, **d), positions)
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()  # [tmax, D]

    def resize(self, tmax):
        """Change the context capacity; the graphs are captured again on the next step."""
        tmax = (tmax + 63) // 64 * 64
        if tmax == self.tmax:
            return
        self.graphs = None
        torch.cuda.synchronize()
        self._alloc(tmax)
        torch.cuda.empty_cache()

    @torch.no_grad()
    def load_kv(self, pk, T):
        assert T < self.tmax, f"context {T} >= tmax {self.tmax}"
        for i in range(self.L):
            k, v = _layer_kv(pk, i)
            self.kc[i][:, :, :T].copy_(k)
            self.vc[i][:, :, :T].copy_(v)
        self.pos = T

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, ids, start=None, chunk=1024):
        """Run tokens `ids` ([T]) at positions start..start+T-1 with the model's modules,
        writing K/V into the static buffers (positions before `start` are reused). Returns
        the logits [1, V] of the last token."""
        from transformers.models.qwen3_moe.modeling_qwen3_moe import apply_rotary_pos_emb

        start = self.pos if start is None else start
        ids = ids.reshape(-1).to(self.dev)
        assert start + ids.numel() <= self.tmax, f"context {start + ids.numel()} > capacity {self.tmax}"
        Hq, Hk, D, G = self.Hq, self.Hk, self.D, self.G
        logits = None
        for c0 in range(0, ids.numel(), chunk):
            part = ids[c0 : c0 + chunk]
            T, s0 = part.numel(), start + c0
            end = s0 + T
            h = self.model.model.embed_tokens(part.view(1, T))
            cos, sin = self.cos[s0:end][None], self.sin[s0:end][None]
            # query t (absolute s0 + t) attends to keys 0 .. s0 + t
            allow = torch.arange(end, device=self.dev)[None] <= torch.arange(s0, end, device=self.dev)[:, None]
            for i, lay in enumerate(self.layers):
                at = lay.self_attn
                xn = lay.input_layernorm(h)
                q = at.q_norm(at.q_proj(xn).view(1, T, Hq, D)).transpose(1, 2)
                k = at.k_norm(at.k_proj(xn).view(1, T, Hk, D)).transpose(1, 2)
                v = at.v_proj(xn).view(1, T, Hk, D).transpose(1, 2)
                q, k = apply_rotary_pos_emb(q, k, cos, sin)
                self.kc[i][:, :, s0:end].copy_(k)
                self.vc[i][:, :, s0:end].copy_(v)
                heads = []
                for j in range(Hk):  # one KV head at a time, float32 attention
                    kk = self.kc[i][:, j : j + 1, :end].float().expand(1, G, end, D)
                    vv = self.vc[i][:, j : j + 1, :end].float().expand(1, G, end, D)
                    qq = q[:, j * G : (j + 1) * G].float()
                    heads.append(F.scaled_dot_product_attention(qq, kk, vv, attn_mask=allow,
                                                                scale=getattr(at, "scaling", D**-0.5)))
                o = torch.cat(heads, 1).to(self.dt).transpose(1, 2).reshape(1, T, Hq * D)
                h = h + at.o_proj(o)
                y = lay.mlp(lay.post_attention_layernorm(h))
                h = h + (y[0] if isinstance(y, tuple) else y)
            logits = self.model.lm_head(self.model.model.norm(h[:, -1:])).view(1, -1)
        self.pos = start + ids.numel()
        return logits

    # ---------------------------------------------------------------- segment bodies
    def _attn_router(self, i, h):
        lay = self.layers[i]
        at, blk = lay.self_attn, lay.mlp
        Hq, Hk, D, H = self.Hq, self.Hk, self.D, self.H
        xn = lay.input_layernorm(h)
        q = at.q_norm(at.q_proj(xn).view(1, 1, Hq, D)).transpose(1, 2)
        k = at.k_norm(at.k_proj(xn).view(1, 1, Hk, D)).transpose(1, 2)
        v = at.v_proj(xn).view(1, 1, Hk, D).transpose(1, 2)
        pos = self.ctl[1:2]
        cos = self.cos.index_select(0, pos).view(1, 1, D)
        sin = self.sin.index_select(0, pos).view(1, 1, D)
        q, k = kernels.rope_decode(q, k, cos, sin)
        self.kc[i].index_copy_(2, pos, k)
        self.vc[i].index_copy_(2, pos, v)
        o = kernels.attn_decode(q, self.kc[i], self.vc[i], pos, getattr(at, "scaling", D**-0.5))
        hm = h + at.o_proj(o.reshape(1, 1, Hq * D))
        xn2 = lay.post_attention_layernorm(hm)
        sel, rw = route(blk.gate(xn2.view(1, H)), self.k, blk.norm_topk, xn2.dtype)
        parts = [sel.float(), rw.float()]
        if self.prefetch:
            ng = getattr(blk, "next_gate", None)
            parts.append(torch.topk(ng(xn2.view(1, H)), self.k, dim=-1).indices.float() if ng is not None
                         else torch.zeros(1, self.k, device=self.dev))
        self.hm.copy_(hm)
        self.xn.copy_(xn2)
        self.row.copy_(torch.cat(parts, 1))

    def _moe(self, i):
        """MoE of layer i from the static buffers -> [1, 1, H]."""
        c = self.rt.cache
        st = c.store
        y = kernels.moe_decode_fast(c.gpu, self.meta_dev, self.xn.view(self.H), self.k, st.n, self.H,
                                    self.layers[i].mlp.I, st.bits, st.group)
        return y.view(1, 1, self.H)

    def _seg(self, j):
        if j == 0:
            h = self.model.model.embed_tokens(self.ctl[0:1].view(1, 1))
        else:
            h = self.hm + self._moe(j - 1)
        if j < self.L:
            self._attn_router(j, h)
        else:
            self.logits.copy_(self.model.lm_head(self.model.model.norm(h)).view(1, -1))

    # ---------------------------------------------------------------- host step of one layer
    def _prepare(self, i, row):
        rt, cache, k = self.rt, self.rt.cache, self.k
        ex = [int(v) for v in row[:k]]
        if rt.recorder is not None:
            import numpy as np

            rt.recorder.append((i, np.array([ex])))
        rt.stats["layer_calls"] += 1
        base = i * self.E
        # ensure + expert copies + meta write + meta copy, in one native call
        slots = cache.prepare_layer([base + e for e in ex], row[k : 2 * k], self.meta_host, self.meta_dev)
        rt.stats["gpu_experts"] += k
        if self.prefetch and i < self.L - 1:
            nb = (i + 1) * self.E
            rt.stats["prefetched"] += cache.prefetch([nb + int(e) for e in set(row[2 * k : 3 * k])], list(slots))

    # ---------------------------------------------------------------- capture / run
    def _cache_key(self):
        c = self.rt.cache
        return (c.gpu.data_ptr(), c.store.bits, self.prefetch)

    @torch.no_grad()
    def capture(self):
        k = self.k
        self.prefetch = bool(getattr(self.rt, "prefetch", False))
        if self.row.shape[1] != (3 if self.prefetch else 2) * k:
            self.row = torch.zeros(1, (3 if self.prefetch else 2) * k, dtype=torch.float32, device=self.dev)
        self.graphs = None
        # the warm-up really runs the segments and writes K/V at ctl[1]: point it at the last
        # slot and restore that slot afterwards, so a capture mid-conversation is harmless
        wp = self.tmax - 1
        saved = [(self.kc[i][:, :, wp].clone(), self.vc[i][:, :, wp].clone()) for i in range(self.L)]
        self.ctl[0] = 0
        self.ctl[1] = wp
        self.meta_host[:k] = torch.arange(k, dtype=torch.float32)
        self.meta_host[k:] = 1.0 / k
        self.meta_dev.copy_(self.meta_host)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                for j in range(self.L + 1):
                    self._seg(j)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for i, (kk, vv) in enumerate(saved):
            self.kc[i][:, :, wp].copy_(kk)
            self.vc[i][:, :, wp].copy_(vv)
        pool = torch.cuda.graph_pool_handle()
        graphs = []
        for j in range(self.L + 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self._seg(j)
            graphs.append(g)
        self.graphs, self._key = graphs, self._cache_key()
        torch.cuda.synchronize()

    def _run(self, j):
        if self.graphs is not None:
            self.graphs[j].replay()
        else:
            self._seg(j)

    @torch.no_grad()
    def next(self, token):
        """token: LongTensor [1] (or [1, 1]) on the device -> logits [1, V] of the next position."""
        assert self.pos < self.tmax, "context full"
        if self.use_graph and (self.graphs is None or self._key != self._cache_key()):
            self.capture()
        self.ctl[0:1].copy_(token.reshape(1))
        self.ctl[1].fill_(self.pos)
        self._run(0)
        for i in range(self.L):
            self._prepare(i, self.row.cpu()[0].tolist())  # the one sync per layer
            self._run(i + 1)
        self.pos += 1
        return self.logits
