"""hipGraph decode of one token at batch 1 for Qwen3-MoE models with paged experts.

Reference interface: wisp/graphdec.py (GraphDecoder(model, rt, tmax, use_graph) with
prefill, load_kv, resize, capture and next; graphdec.py:35-308).

A decode step needs one host decision per MoE layer (which experts to page into the slot
pool), so it is cut at those L paging points into L + 1 segments, each captured once as a
hipGraph and replayed every token:

    segment 0      token embedding -> attention(0) -> router(0)       -> route row
    host step i    route row -> expert cache (native LRU + page kernel) -> meta_dev
    segment i      MoE(i-1) -> residual -> attention(i) -> router(i)  -> route row
    segment L      MoE(L-1) -> residual -> final norm -> lm_head      -> logits

How this build lays it out:
  * DecodeShape reads the dimensions and every per-layer weight once, and checks them
    against what the decode kernels take (bias-free projections, Qwen3 q/k head norms,
    contiguous weights of the embedding's dtype on its device).
  * K/V of all layers is ONE allocation [L, 2, Hk, cap + 64, D]; kc[i] / vc[i] are views
    [1, Hk, cap + 64, D]. The 64 positions past the capacity are a scratch area: the
    capture's warm-up runs the segments at position `cap`, where nothing is ever attended
    (attention reads positions <= pos < cap), so capturing needs no save and restore of
    live K/V.
  * Every tensor a segment reads or writes exists once (token/position in `ctl`, the
    residual streams, q/k/v, router logits, route row, meta), so the segments' kernel
    arguments never change and the graphs follow the device-side position and routing.
  * A segment is eight launches per layer, all this package's gfx950 kernels: RMSNorm +
    q/k/v GEMV, attention over the static cache with the q/k head norm + rope + K/V store
    folded into its first launch (two), o_proj + residual, RMSNorm + router GEMV, route,
    and the two MoE decode kernels.
  * Host step: the route kernel writes the row and bumps a sequence flag in pinned
    memory; one native call waits for the flag, runs the cache's LRU step, queues the
    page kernel for the misses and writes meta on the stream -- no stream sync per layer.
    With prefetch or a routing recorder the row is read back instead (one sync per layer).
  * Device paging (the default where the cache allows it: LRU policy, page-kernel copies):
    the paging point itself runs on the GPU (one kernel takes the router's top-k and runs
    the cache's LRU step on it, then the page kernel copies the misses), so the L + 1
    segments and the L paging points are captured as ONE graph per token and the host
    only writes the token and position and replays it. The bookkeeping is the same LRU
    step; the cache copies its state back to the host core when the host next needs it.
  * Prefill runs the model's own modules over chunks of tokens, attention in float32 over
    the static cache with the KV heads repeated for their query groups; K/V are written
    straight into the static buffers.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import kernels

SCRATCH = 64  # positions past the capacity: where the capture's warm-up writes K/V


def _kv_of(past, i):
    """(keys, values) [1, Hk, T, D] of layer i from a transformers cache (a DynamicCache with
    per-layer objects, an older one with key/value lists, or a tuple of per-layer pairs)."""
    layers = getattr(past, "layers", None)
    if layers is not None:
        return layers[i].keys, layers[i].values
    if hasattr(past, "key_cache"):
        return past.key_cache[i], past.value_cache[i]
    k, v = past[i][0], past[i][1]
    return k, v


class DecodeShape:
    """Dimensions and per-layer weights of an all-MoE Qwen3 model, as the decode kernels
    take them."""

    def __init__(self, model):
        cfg = model.config
        self.cfg = cfg
        self.L, self.H = cfg.num_hidden_layers, cfg.hidden_size
        self.Hq, self.Hk = cfg.num_attention_heads, cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or self.H // self.Hq
        self.G = self.Hq // self.Hk
        self.layers = list(model.model.layers)
        if not all(hasattr(lay.mlp, "top_k") for lay in self.layers):
            raise AssertionError("GraphDecoder needs an all-MoE model (paged MoE blocks in every layer)")
        first = self.layers[0].mlp
        self.k = first.top_k
        self.E = getattr(first, "E", None) or cfg.num_experts
        emb = model.model.embed_tokens.weight
        self.dev, self.dt = emb.device, emb.dtype
        if self.dev.type != "cuda":
            raise RuntimeError("GraphDecoder runs the gfx950 decode kernels: the model must be on a ROCm device")
        self.per_layer = [self._layer_weights(lay) for lay in self.layers]
        norm = model.model.norm
        self.w_final, self.eps_final = norm.weight, norm.variance_epsilon
        self.w_embed, self.w_head = emb, model.lm_head.weight

    def _layer_weights(self, lay):
        at, blk = lay.self_attn, lay.mlp
        for name, lin in (("q_proj", at.q_proj), ("k_proj", at.k_proj), ("v_proj", at.v_proj),
                          ("o_proj", at.o_proj), ("router", blk.gate)):
            if getattr(lin, "bias", None) is not None:
                raise AssertionError(f"the decode kernels take bias-free projections (Qwen3-MoE); {name} has one")
        if not (hasattr(at, "q_norm") and hasattr(at, "k_norm")):
            raise AssertionError("the decode kernels take Qwen3-style attention with q_norm / k_norm")
        w = dict(ln1=lay.input_layernorm.weight, eps1=lay.input_layernorm.variance_epsilon,
                 q=at.q_proj.weight, k=at.k_proj.weight, v=at.v_proj.weight, o=at.o_proj.weight,
                 qn=at.q_norm.weight, kn=at.k_norm.weight, epsq=at.q_norm.variance_epsilon,
                 ln2=lay.post_attention_layernorm.weight, eps2=lay.post_attention_layernorm.variance_epsilon,
                 gate=blk.gate.weight, scale=getattr(at, "scaling", self.D**-0.5), norm_topk=blk.norm_topk,
                 I=blk.I)
        for key in ("ln1", "q", "k", "v", "o", "qn", "kn", "ln2", "gate"):
            t = w[key]
            if t.dtype != self.dt or not t.is_contiguous() or t.device != self.dev:
                raise AssertionError(f"the decode kernels need contiguous {self.dt} weights on {self.dev} ({key})")
        return w


class GraphDecoder:
    def __init__(self, model, rt=None, tmax=2048, use_graph=True, device_paging="auto"):
        """device_paging: "auto" = page on the GPU when the cache can (LRU policy, page-kernel
        copies, no prefetch or routing recorder), True = require it, False = host steps."""
        assert device_paging in ("auto", True, False), device_paging
        s = DecodeShape(model)
        self.shape, self.model, self.rt = s, model, rt
        self.L, self.H, self.Hq, self.Hk, self.D, self.G = s.L, s.H, s.Hq, s.Hk, s.D, s.G
        self.k, self.E, self.layers = s.k, s.E, s.layers
        self.dev, self.dt = s.dev, s.dt
        self.use_graph = use_graph
        self.device_paging = device_paging
        self._dev = False  # this capture pages on the GPU
        self._ids_dev = self._ids_ring = None
        self.graphs, self._key = None, None
        self.pos = 0
        self.kv = None
        self._kv_alloc((tmax + 63) // 64 * 64)
        bf = dict(device=self.dev, dtype=self.dt)
        f32 = dict(device=self.dev, dtype=torch.float32)
        self.ctl = torch.zeros(2, dtype=torch.long, device=self.dev)  # [token, position]
        self.hbuf = torch.zeros(self.H, **bf)  # residual stream entering attention
        self.hm = torch.zeros(1, 1, self.H, **bf)  # residual stream after attention
        self.xn = torch.zeros(1, 1, self.H, **bf)  # normed MoE input
        self.qkv = torch.zeros((self.Hq + 2 * self.Hk) * self.D, **bf)
        self.rlogits = torch.zeros(self.E, **bf)
        self.logits = torch.zeros(1, s.cfg.vocab_size, **bf)
        self.prefetch = bool(rt is not None and getattr(rt, "prefetch", False))
        self.row = torch.zeros(1, self._row_len(), **f32)  # [expert ids | weights (| predicted next)]
        self.meta_dev = torch.zeros(2 * self.k, **f32)  # [slot ids | weights] the MoE kernels read
        self.meta_host = torch.zeros(2 * self.k, dtype=torch.float32, pin_memory=True)
        self.row_host = torch.zeros(3 * self.k, dtype=torch.float32, pin_memory=True)
        self.flag_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.seq_dev = torch.zeros(1, dtype=torch.int32, device=self.dev)

    def _row_len(self):
        return (3 if self.prefetch else 2) * self.k

    # ---------------------------------------------------------------- static K/V
    def _kv_alloc(self, cap):
        """K/V for `cap` positions (+ the scratch area), keeping positions < min(pos, cap)."""
        keep = min(self.pos, cap)
        kv = torch.zeros(self.L, 2, self.Hk, cap + SCRATCH, self.D, device=self.dev, dtype=self.dt)
        if self.kv is not None and keep:
            kv[:, :, :, :keep].copy_(self.kv[:, :, :, :keep])
        self.kv = kv
        self.kc = [kv[i, 0].unsqueeze(0) for i in range(self.L)]  # [1, Hk, cap + SCRATCH, D]
        self.vc = [kv[i, 1].unsqueeze(0) for i in range(self.L)]
        self.tmax, self.pos = cap, keep
        positions = torch.arange(cap + SCRATCH, device=self.dev)[None]
        probe = torch.zeros(1, 1, self.H, device=self.dev, dtype=self.dt)
        cos, sin = self.model.model.rotary_emb(probe, positions)
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()  # [cap + SCRATCH, D]

    def resize(self, tmax):
        """Change the context capacity, keeping the K/V already written; the graphs are
        captured again on the next step."""
        cap = (tmax + 63) // 64 * 64
        if cap == self.tmax:
            return
        self.graphs = None
        torch.cuda.synchronize(self.dev)
        self._kv_alloc(cap)
        torch.cuda.empty_cache()

    @torch.no_grad()
    def load_kv(self, pk, T):
        """Take positions 0 .. T-1 of every layer's K/V from a transformers cache."""
        assert T < self.tmax, f"context {T} >= tmax {self.tmax}"
        for i in range(self.L):
            k, v = _kv_of(pk, i)
            self.kv[i, 0, :, :T].copy_(k[0])
            self.kv[i, 1, :, :T].copy_(v[0])
        self.pos = T

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, ids, start=None, chunk=1024):
        """Run tokens `ids` ([T]) at positions start .. start+T-1 through the model's modules
        and the paged MoE blocks, writing K/V into the static buffers (positions before
        `start` are kept and attended). Returns the logits [1, V] of the last token."""
        from transformers.models.qwen3_moe.modeling_qwen3_moe import apply_rotary_pos_emb

        start = self.pos if start is None else start
        ids = ids.reshape(-1).to(self.dev)
        total = start + ids.numel()
        assert total <= self.tmax, f"context {total} > capacity {self.tmax}"
        Hq, Hk, D = self.Hq, self.Hk, self.D
        embed, final, head = self.model.model.embed_tokens, self.model.model.norm, self.model.lm_head
        logits = None
        for c0 in range(0, ids.numel(), chunk):
            toks = ids[c0 : c0 + chunk]
            T, s0 = toks.numel(), start + c0
            s1 = s0 + T
            cos, sin = self.cos[s0:s1][None], self.sin[s0:s1][None]
            # query s0 + t sees keys 0 .. s0 + t
            causal = torch.arange(s1, device=self.dev)[None, :] <= torch.arange(s0, s1, device=self.dev)[:, None]
            h = embed(toks.view(1, T))
            for i, lay in enumerate(self.layers):
                at = lay.self_attn
                xn = lay.input_layernorm(h)
                q = at.q_norm(at.q_proj(xn).view(1, T, Hq, D)).transpose(1, 2)
                kk = at.k_norm(at.k_proj(xn).view(1, T, Hk, D)).transpose(1, 2)
                vv = at.v_proj(xn).view(1, T, Hk, D).transpose(1, 2)
                q, kk = apply_rotary_pos_emb(q, kk, cos, sin)
                self.kv[i, 0, :, s0:s1].copy_(kk[0])
                self.kv[i, 1, :, s0:s1].copy_(vv[0])
                # float32 attention over the cache, each KV head repeated for its query group
                keys = self.kv[i, 0, :, :s1].float().repeat_interleave(self.G, dim=0)[None]
                vals = self.kv[i, 1, :, :s1].float().repeat_interleave(self.G, dim=0)[None]
                o = F.scaled_dot_product_attention(q.float(), keys, vals, attn_mask=causal,
                                                   scale=self.shape.per_layer[i]["scale"])
                h = h + at.o_proj(o.to(self.dt).transpose(1, 2).reshape(1, T, Hq * D))
                y = lay.mlp(lay.post_attention_layernorm(h))
                h = h + (y[0] if isinstance(y, tuple) else y)
            logits = head(final(h[:, -1:])).view(1, -1)
        self.pos = total
        return logits

    # ---------------------------------------------------------------- segment bodies
    def _attention_router(self, i, a, a_row=None, b=None):
        """Layer i from the residual stream h = a (+ b) (a_row: token row of the embedding):
        RMSNorm + q/k/v, q/k head norm + rope + K/V store, attention, o_proj + residual,
        RMSNorm + router, route. Leaves h + attention in hm, the MoE input in xn and the
        route row in row (and, for the host, in row_host with the flag bumped)."""
        w, Hq, Hk, D, H = self.shape.per_layer[i], self.Hq, self.Hk, self.D, self.H
        pos = self.ctl[1:2]
        kernels.dl_gemv(self.qkv, w["q"], a, w1=w["k"], w2=w["v"], a_row=a_row, b=b, norm_w=w["ln1"],
                        eps=w["eps1"], h_out=self.hbuf)
        attn = kernels.dl_qk_rope_attn(self.qkv, w["qn"], w["kn"], w["epsq"], self.cos, self.sin, pos, Hq, Hk, D,
                                       self.kc[i], self.vc[i], w["scale"])
        kernels.dl_gemv(self.hm.view(H), w["o"], attn.view(Hq * D), res=self.hbuf)
        kernels.dl_gemv(self.rlogits, w["gate"], self.hm.view(H), norm_w=w["ln2"], eps=w["eps2"],
                        x_out=self.xn.view(H))
        if not self._dev:  # (device paging: routed by the paging point's kernel, _device_step)
            kernels.dl_route(self.rlogits, self.k, w["norm_topk"], self.row.view(-1), self.row_host, self.flag_host,
                             self.seq_dev)
        if self.prefetch:  # the next layer's router on this layer's input predicts its experts
            nxt = getattr(self.layers[i].mlp, "next_gate", None)
            guess = (torch.topk(nxt(self.xn.view(1, H)), self.k, dim=-1).indices.float() if nxt is not None
                     else torch.zeros(1, self.k, device=self.dev))
            self.row[:, 2 * self.k :].copy_(guess)

    def _moe(self, i):
        """The MoE output [H] of layer i on xn with the routing in meta_dev. Overridable, as
        the reference's (graphdec.py:189-197): an override returns any contiguous tensor of
        H values of the model's dtype."""
        cache = self.rt.cache
        st = cache.store
        return kernels.moe_decode_fast(cache.gpu, self.meta_dev, self.xn.view(self.H), self.k, st.n, self.H,
                                       self.shape.per_layer[i]["I"], st.bits, st.group)

    def _segment(self, j):
        if j == 0:  # h = embedding row of the token
            a, a_row, b = self.shape.w_embed, self.ctl[0:1], None
        else:  # h = hm + MoE(j - 1)
            a, a_row, b = self.hm.view(self.H), None, self._moe(j - 1)
        if j < self.L:
            self._attention_router(j, a, a_row, b)
        else:
            kernels.dl_gemv(self.logits.view(-1), self.shape.w_head, a, a_row=a_row, b=b,
                            norm_w=self.shape.w_final, eps=self.shape.eps_final)

    # ---------------------------------------------------------------- paging point on the GPU
    def _forced_ids(self):
        """True when a subclass replaces the router's expert ids (_expert_ids)."""
        return type(self)._expert_ids is not GraphDecoder._expert_ids

    def _device_ok(self):
        """Whether this step pages on the GPU; starts device paging on the cache if so."""
        rt = self.rt
        if (self.device_paging is False or rt is None or self.prefetch or rt.recorder is not None
                or self._custom_prepare()):
            if self.device_paging is True:
                raise RuntimeError("device paging needs a runtime without prefetch, a routing recorder or a "
                                   "_prepare override")
            return False
        dyn = rt.cache.nslots - getattr(rt.cache, "n_static", 0)
        if dyn < self.k:  # the host steps' core refuses it as well, on the first miss
            raise RuntimeError(f"the cache has {dyn} dynamic slots, fewer than top-k = {self.k}: no evictable slot")
        try:
            rt.cache.device_begin()
        except RuntimeError:
            if self.device_paging is True:
                raise
            return False
        return True

    def _device_step(self, i):
        """Layer i's routing and paging point on the current stream, one launch + the page
        kernel: the router's top-k of rlogits into row, the LRU step of those experts (or of
        the forced ids), meta_dev written, misses paged."""
        ids = self._ids_dev[i] if self._ids_dev is not None else None
        self.rt.cache.device_route_step(self.rlogits, self.k, self.shape.per_layer[i]["norm_topk"], self.row.view(-1),
                                        ids, i * self.E, self.E, self.meta_dev)

    def _stage_ids(self):
        """Forced expert ids of every layer for this token -> _ids_dev (pinned ring, so the
        host can run ahead of the GPU by a few tokens); -1 (the router's choice) for a layer
        whose _expert_ids is None."""
        buf, ev = self._ids_ring[self._ids_next]
        ev.synchronize()  # the copy that last read this buffer has run
        for i in range(self.L):
            ids = self._expert_ids(i)
            if ids is None:
                buf[i].fill_(-1)
            else:
                buf[i].copy_(torch.as_tensor(ids, dtype=torch.int64))
        self._ids_dev.copy_(buf, non_blocking=True)
        ev.record()
        self._ids_next = (self._ids_next + 1) % len(self._ids_ring)

    # ---------------------------------------------------------------- host step of one layer
    def _expert_ids(self, i):
        """Expert ids of layer i replacing the router's choice (int64 [k]), or None for the
        router's own. A hook for synthetic routing; the weights stay the router's."""
        return None

    def _custom_prepare(self):
        """True when a subclass replaces the host step (_prepare)."""
        return type(self)._prepare is not GraphDecoder._prepare

    def _prepare(self, i, row):
        """Host step of layer i from the route row read back to the host (row: the list
        [expert ids | weights (| predicted next ids)] of floats): page the experts (or the
        _expert_ids hook's), write meta_dev, prefetch the predicted ones, count the step.
        The reference's overridable host step (graphdec.py:216-234): a subclass that
        overrides it owns the whole step; the decoder then reads the row back every layer
        (one sync per layer) and pages nothing itself, as with prefetch or a recorder."""
        rt, cache, k = self.rt, self.rt.cache, self.k
        ex = [int(v) for v in row[:k]]
        forced = self._expert_ids(i)
        if forced is not None:
            ex = [int(v) for v in forced]
        if rt.recorder is not None:
            import numpy as np

            rt.recorder.append((i, np.array([ex])))
        base = i * self.E
        slots = cache.prepare_layer([base + e for e in ex], row[k : 2 * k], self.meta_host, self.meta_dev)
        if self.prefetch and i + 1 < self.L:
            nxt = (i + 1) * self.E
            rt.stats["prefetched"] += cache.prefetch([nxt + int(e) for e in set(row[2 * k : 3 * k])], list(slots))
        rt.stats["layer_calls"] += 1
        rt.stats["gpu_experts"] += k

    # ---------------------------------------------------------------- capture / replay
    def _cache_key(self):
        if self.rt is None:  # (a _prepare / _moe override owns the experts)
            return (None, self.prefetch, self.device_paging)
        cache = self.rt.cache
        return (id(cache), cache.gpu.data_ptr(), cache.nslots, cache.store.bits, self.prefetch, self.device_paging,
                self.rt.recorder is not None)

    @torch.no_grad()
    def capture(self):
        """Run every segment twice eagerly at the scratch position (first use of each kernel,
        allocations of the graph pool's shapes), then capture the L + 1 segments."""
        self.prefetch = bool(getattr(self.rt, "prefetch", False))
        if self.row.shape[1] != self._row_len():
            self.row = torch.zeros(1, self._row_len(), dtype=torch.float32, device=self.dev)
        self.graphs = None
        self._dev = self._device_ok()
        if self._dev and self._forced_ids():
            self._ids_dev = torch.zeros(self.L, self.k, dtype=torch.int64, device=self.dev)
            self._ids_ring = [(torch.zeros(self.L, self.k, dtype=torch.int64, pin_memory=True), torch.cuda.Event())
                              for _ in range(4)]
            self._ids_next = 0
        else:
            self._ids_dev = self._ids_ring = None
        k = self.k
        self.ctl[0] = 0
        self.ctl[1] = self.tmax  # scratch: never attended by a real position
        self.meta_dev[:k] = torch.arange(k, dtype=torch.float32, device=self.dev)  # any resident slots
        self.meta_dev[k:] = 1.0 / k
        torch.cuda.synchronize(self.dev)
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                for j in range(self.L + 1):
                    self._segment(j)
            if self._dev:  # the paging point's kernels once, without a step
                self.rt.cache.device_route_step(self.rlogits, 0, True, self.row.view(-1), None, 0, self.E,
                                                self.meta_dev)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        torch.cuda.synchronize(self.dev)
        pool = torch.cuda.graph_pool_handle()
        graphs = []
        if self._dev:  # one graph: segments and paging points
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                for j in range(self.L + 1):
                    self._segment(j)
                    if j < self.L:
                        self._device_step(j)
            graphs.append(g)
        else:
            for j in range(self.L + 1):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool):
                    self._segment(j)
                graphs.append(g)
        self.graphs, self._key = graphs, self._cache_key()
        torch.cuda.synchronize(self.dev)

    def _replay(self, j):
        if self.graphs is None:
            self._segment(j)
        else:
            self.graphs[j].replay()

    @torch.no_grad()
    def next(self, token):
        """token: LongTensor [1] (or [1, 1]) on the device -> logits [1, V] of the next position."""
        assert self.pos < self.tmax, "context full"
        if self.use_graph and (self.graphs is None or self._key != self._cache_key()):
            self.capture()
        if not self.use_graph:
            self._dev = self._device_ok()
            if self._dev and self._forced_ids() and self._ids_ring is None:
                self._ids_dev = torch.zeros(self.L, self.k, dtype=torch.int64, device=self.dev)
                self._ids_ring = [(torch.zeros(self.L, self.k, dtype=torch.int64, pin_memory=True),
                                   torch.cuda.Event()) for _ in range(4)]
                self._ids_next = 0
        elif self._dev:
            self.rt.cache.device_begin()  # again, if a host-side cache call ended it
        self.ctl[0:1].copy_(token.reshape(1))
        self.ctl[1].fill_(self.pos)
        rt = self.rt
        if self._dev:  # the whole step on the GPU
            if self._ids_dev is not None:
                self._stage_ids()
            if self.graphs is not None:
                self.graphs[0].replay()
            else:
                for j in range(self.L + 1):
                    self._segment(j)
                    if j < self.L:
                        self._device_step(j)
            rt.stats["layer_calls"] += self.L
            rt.stats["gpu_experts"] += self.L * self.k
            self.pos += 1
            return self.logits
        custom = self._custom_prepare()
        if rt is None and not custom:
            raise RuntimeError("a decoder without a runtime needs _prepare and _moe overrides")
        signalled = not (custom or self.prefetch or rt.recorder is not None)
        flag = int(self.flag_host[0])  # no route kernel is in flight here
        self._replay(0)
        for i in range(self.L):
            if signalled:  # wait for the route kernel's row in host memory; page; write meta
                flag = rt.cache.prepare_signaled(self.row_host, self.flag_host, flag, i * self.E, self.k, self.E,
                                                 self._expert_ids(i), self.meta_host, self.meta_dev)
                rt.stats["layer_calls"] += 1
                rt.stats["gpu_experts"] += self.k
            else:
                self._prepare(i, self.row.cpu()[0].tolist())  # the one sync of this layer
            self._replay(i + 1)
        self.pos += 1
        return self.logits
