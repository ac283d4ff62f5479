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
length. The decode segments run only this package's gfx950 kernels, nine launches per
layer: RMSNorm + q/k/v projection, q/k head norm + rope + KV store, grouped attention
over the static cache (two), o_proj + residual, RMSNorm + router gate, route, and the
two MoE decode kernels on the expert cache's slot pool (the model's modules would be
about sixty small kernels per layer at batch 1). Prefill runs the model's own modules in chunks, with
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
        self.row_host = torch.zeros(3 * self.k, dtype=torch.float32, pin_memory=True)
        # the route kernel also writes the row here and bumps the flag (no stream sync per layer)
        self.flag_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.seq_dev = torch.zeros(1, dtype=torch.int32, device=self.dev)
        self.graphs, self._key = None, None
        self._dense_setup(cfg)

    def _dense_setup(self, cfg):
        """Weights and static buffers of the fused decode segments (csrc/decode_layer.hip):
        per layer the input/post-attention RMSNorm weights, q/k/v/o, q_norm/k_norm and the
        router gate, all bf16 and contiguous as the modules hold them."""
        Hq, Hk, D, H = self.Hq, self.Hk, self.D, self.H
        W = []
        for lay in self.layers:
            at, blk = lay.self_attn, lay.mlp
            for lin in (at.q_proj, at.k_proj, at.v_proj, at.o_proj, blk.gate):
                if getattr(lin, "bias", None) is not None:
                    raise AssertionError("GraphDecoder's decode kernels take bias-free projections (Qwen3-MoE)")
            if not (hasattr(at, "q_norm") and hasattr(at, "k_norm")):
                raise AssertionError("GraphDecoder's decode kernels take Qwen3-style attention (q_norm, k_norm)")
            W.append(dict(
                ln1=lay.input_layernorm.weight, eps1=lay.input_layernorm.variance_epsilon,
                q=at.q_proj.weight, k=at.k_proj.weight, v=at.v_proj.weight, o=at.o_proj.weight,
                qn=at.q_norm.weight, kn=at.k_norm.weight, epsq=at.q_norm.variance_epsilon,
                ln2=lay.post_attention_layernorm.weight, eps2=lay.post_attention_layernorm.variance_epsilon,
                gate=blk.gate.weight, scale=getattr(at, "scaling", D**-0.5), norm_topk=blk.norm_topk,
            ))
        for w in W:
            for key in ("ln1", "q", "k", "v", "o", "qn", "kn", "ln2", "gate"):
                t = w[key]
                if t.dtype != self.dt or not t.is_contiguous() or t.device != self.dev:
                    raise AssertionError(f"decode kernels need contiguous {self.dt} weights on {self.dev} ({key})")
        self.W = W
        nrm = self.model.model.norm
        self.w_final, self.eps_final = nrm.weight, nrm.variance_epsilon
        self.w_embed, self.w_head = self.model.model.embed_tokens.weight, self.model.lm_head.weight
        d = dict(device=self.dev, dtype=self.dt)
        self.hbuf = torch.zeros(H, **d)  # residual stream before attention (h)
        self.qkv = torch.zeros((Hq + 2 * Hk) * D, **d)
        self.qo = torch.zeros(Hq * D, **d)
        self.rlogits = torch.zeros(self.E, **d)

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
    def _attn_router(self, i, a, a_row=None, b=None):
        """Attention and router of layer i on h = a (+ b), graphdec.py:160-192, as six
        launches: RMSNorm + q/k/v (one GEMV), q/k head norm + rope + KV store, attention
        (two), o_proj + residual, RMSNorm + router gate, route. Leaves h + attention in hm,
        the MoE input in xn and [expert ids | weights] in row."""
        w, Hq, Hk, D, H = self.W[i], self.Hq, self.Hk, self.D, self.H
        pos = self.ctl[1:2]
        kernels.dl_gemv(self.qkv, w["q"], a, w1=w["k"], w2=w["v"], a_row=a_row, b=b, norm_w=w["ln1"],
                        eps=w["eps1"], h_out=self.hbuf)
        kernels.dl_qk_rope(self.qkv, w["qn"], w["kn"], w["epsq"], self.cos, self.sin, pos, Hq, Hk, D,
                           self.kc[i], self.vc[i], self.qo)
        o = kernels.attn_decode(self.qo.view(Hq, D), self.kc[i], self.vc[i], pos, w["scale"])
        kernels.dl_gemv(self.hm.view(H), w["o"], o.view(Hq * D), res=self.hbuf)
        kernels.dl_gemv(self.rlogits, w["gate"], self.hm.view(H), norm_w=w["ln2"], eps=w["eps2"],
                        x_out=self.xn.view(H))
        kernels.dl_route(self.rlogits, self.k, w["norm_topk"], self.row.view(-1), self.row_host, self.flag_host,
                         self.seq_dev)
        if self.prefetch:
            ng = getattr(self.layers[i].mlp, "next_gate", None)
            pred = (torch.topk(ng(self.xn.view(1, H)), self.k, dim=-1).indices.float() if ng is not None
                    else torch.zeros(1, self.k, device=self.dev))
            self.row[:, 2 * self.k :].copy_(pred)

    def _moe(self, i):
        """MoE of layer i from the static buffers -> [H]."""
        c = self.rt.cache
        st = c.store
        return kernels.moe_decode_fast(c.gpu, self.meta_dev, self.xn.view(self.H), self.k, st.n, self.H,
                                       self.layers[i].mlp.I, st.bits, st.group)

    def _seg(self, j):
        if j == 0:  # h = embed_tokens(token)
            a, a_row, b = self.w_embed, self.ctl[0:1], None
        else:  # h = hm + MoE(j - 1)
            a, a_row, b = self.hm.view(self.H), None, self._moe(j - 1)
        if j < self.L:
            self._attn_router(j, a, a_row, b)
        else:
            kernels.dl_gemv(self.logits.view(-1), self.w_head, a, a_row=a_row, b=b, norm_w=self.w_final,
                            eps=self.eps_final)

    # ---------------------------------------------------------------- host step of one layer
    def _expert_ids(self, i):
        """Expert ids of layer i replacing the router's choice (int64 [k]), or None for the
        router's own. A hook for synthetic routing; the weights stay the router's."""
        return None

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
        rt = self.rt
        fast = not self.prefetch and rt.recorder is None
        flag = int(self.flag_host[0])  # no route kernel is in flight here
        self._run(0)
        for i in range(self.L):
            if fast:  # wait for the row the route kernel writes to host memory, then ensure / copy / meta
                flag = rt.cache.prepare_signaled(self.row_host, self.flag_host, flag, i * self.E, self.k, self.E,
                                                 self._expert_ids(i), self.meta_host, self.meta_dev)
                rt.stats["layer_calls"] += 1
                rt.stats["gpu_experts"] += self.k
            else:
                self._prepare(i, self.row.cpu()[0].tolist())  # the one sync per layer
            self._run(i + 1)
        self.pos += 1
        return self.logits
